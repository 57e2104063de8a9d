"""Errors raised by oops_amd operators.

Same contract as the reference's ``OOpsUnsupportedError`` (oops/_errors.py:28) and
``unsupported()`` message builder (oops/runtime/dispatch.py:514-526): a
``NotImplementedError`` subclass for unsupported devices, dtypes, layouts,
launch limits or differentiation modes; malformed argument relationships raise
``ValueError`` instead.
"""

from __future__ import annotations


class OOpsUnsupportedError(NotImplementedError):
    """An operator cannot serve the requested execution contract."""


def unsupported(operator: str, reason: str, **context: object) -> OOpsUnsupportedError:
    """Build an ``OOpsUnsupportedError`` with ``(key=value, ...)`` context appended."""

    suffix = ""
    if context:
        suffix = " (" + ", ".join(f"{key}={value}" for key, value in context.items()) + ")"
    return OOpsUnsupportedError(f"{operator} {reason}{suffix}")
