"""Fixed-order sums of float32 partial arrays over their leading axis, many arrays per launch.

The backward kernels write float32 partials (one row per workgroup or per K-chunk) where the
reference sums its partials with torch reductions (for triangle_multiplication:
oops/pair/triangle_multiplication/triton/generic.py:824, :1017-1018, :1092, :1115).  ``PartialSums``
collects such arrays and sums all of them with one ``oops_sum_partials`` launch.
"""

from __future__ import annotations

import ctypes

import torch
from torch import Tensor

from . import _lib

_OUT_DTYPE = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}


class PartialSums:
    """``add`` registers ``parts`` (P, *shape) float32 and returns the (still unwritten) ``shape`` result in
    ``dtype`` (or in the given contiguous ``out``); ``run`` sums every registered array (one launch per
    SUM_MAX_SEGMENTS arrays, two when an array has more than 256 rows)."""

    def __init__(self) -> None:
        self._segs: list[tuple[Tensor, Tensor]] = []

    def add(self, parts: Tensor, dtype: torch.dtype = torch.float32, out: Tensor | None = None) -> Tensor:
        if parts.dtype != torch.float32 or parts.dim() < 1:
            raise TypeError("partial sums take float32 arrays with a leading parts axis")
        n = 1
        for d in parts.shape[1:]:
            n *= d
        rows = parts.reshape(parts.shape[0], n)
        if rows.numel() and rows.stride(1) != 1:
            rows = rows.contiguous()
        if out is None:
            out = torch.empty(parts.shape[1:], dtype=dtype, device=parts.device)
        elif not out.is_contiguous() or out.numel() != rows.shape[1]:
            raise ValueError("a partial-sum destination must be contiguous with one value per column")
        self._segs.append((rows, out))
        return out

    def run(self, stream: int) -> None:
        lib = _lib.load()
        for i in range(0, len(self._segs), _lib.SUM_MAX_SEGMENTS):
            chunk = self._segs[i : i + _lib.SUM_MAX_SEGMENTS]
            arr = (_lib.SumSegment * len(chunk))()
            for seg, (rows, out) in zip(arr, chunk):
                seg.parts = rows.data_ptr() if rows.numel() else None
                seg.out = out.data_ptr() if out.numel() else None
                seg.count = rows.shape[0]
                seg.n = rows.shape[1]
                seg.part_stride = rows.stride(0) if rows.shape[0] > 1 else rows.shape[1]
                seg.out_dtype = _OUT_DTYPE[out.dtype]
            ws_bytes = lib.oops_sum_partials_workspace_bytes(arr, len(chunk))
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=chunk[0][1].device) if ws_bytes else None
            rc = lib.oops_sum_partials(arr, len(chunk), None if ws is None else ws.data_ptr(), ws_bytes,
                                       ctypes.c_void_p(stream))  # fmt: skip
            _lib.check(rc, "partial sums")
        self._segs.clear()
