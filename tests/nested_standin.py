"""Test-only stand-in for DanLing's ``NestedTensor`` (danling >= 0.4.6, not installed here).

It implements the subset of the packing protocol the reference's nested
attention paths use (oops/attention/triangle/triangle_attention.py:261-513,
oops/attention/triangle/nested.py:20-120, tests/attention/triangle/
test_triangle_attention.py:65-169):

* ``NestedTensor(tensors, ragged_dims=...)``: every element has the same rank;
  the ``ragged_dims`` of each element are flattened (in the listed order) into
  one packed axis, followed by the remaining element dims in natural order:
  ``packed_dim_order = (*ragged_dims, *others)``.  ``.concat`` concatenates the
  packed elements along that axis.
* ``.packed_offsets()``: boundaries of the elements on the packed axis.
* ``.ragged_level_offsets(level)``: cumulative sizes of ragged dim ``level``.
* ``.transpose(a, b)``: swaps two element dims as a view of the same packed
  storage (ragged dims and packing order are renamed, ``concat`` unchanged).
* ``.packed_like(values)``: same topology over new packed values;
  ``.packed_with_static_tail(values)`` the same with other static dims.
* ``.element_sizes()``: each element's shape.
* ``torch.unbind(nested)``: the elements as dense tensors (differentiable).
"""

from __future__ import annotations

from math import prod

import torch


class NestedTensor:
    def __init__(self, tensors=None, *, ragged_dims, packed_dim_order=None, _sizes=None, _concat=None):
        if tensors is not None:
            _sizes = [tuple(t.shape) for t in tensors]
        rank = len(_sizes[0])
        assert all(len(s) == rank for s in _sizes)
        self.ragged_dims = tuple(int(d) for d in ragged_dims)
        if packed_dim_order is None:
            packed_dim_order = (*self.ragged_dims, *(d for d in range(rank) if d not in self.ragged_dims))
        self.packed_dim_order = tuple(packed_dim_order)
        self._sizes = [tuple(s) for s in _sizes]
        self.batch_first = True
        if _concat is None:
            _concat = torch.cat([self._pack(t) for t in tensors])
        self.concat = _concat

    # ---------------------------------------------------------------- layout
    def _pack(self, element):
        order = self.packed_dim_order
        nr = len(self.ragged_dims)
        moved = element.permute(order)
        return moved.reshape(-1, *moved.shape[nr:])

    def dim(self):
        return len(self._sizes[0]) + 1

    def element_sizes(self):
        return list(self._sizes)

    def packed_offsets(self, dtype=torch.int64, device=None):
        counts = [prod(s[d] for d in self.ragged_dims) for s in self._sizes]
        return torch.tensor([0, *torch.tensor(counts).cumsum(0).tolist()], dtype=dtype, device=device)

    def ragged_level_offsets(self, level, dtype=torch.int64, device=None):
        d = self.ragged_dims[level]
        counts = [s[d] for s in self._sizes]
        return torch.tensor([0, *torch.tensor(counts).cumsum(0).tolist()], dtype=dtype, device=device)

    def packed_like(self, values):
        if tuple(values.shape) != tuple(self.concat.shape):
            raise ValueError(f"packed_like: values {tuple(values.shape)} != {tuple(self.concat.shape)}")
        return NestedTensor(
            ragged_dims=self.ragged_dims, packed_dim_order=self.packed_dim_order, _sizes=self._sizes, _concat=values
        )

    def packed_with_static_tail(self, values):
        """Same ragged topology over packed values whose static (non-ragged) dims differ."""

        nr = len(self.ragged_dims)
        static_dims = self.packed_dim_order[nr:]
        if values.shape[0] != self.concat.shape[0] or values.dim() - 1 != len(static_dims):
            raise ValueError("packed_with_static_tail: packed axis or static rank differs")
        sizes = []
        for s in self._sizes:
            s = list(s)
            for d, n in zip(static_dims, values.shape[1:]):
                s[d] = n
            sizes.append(tuple(s))
        return NestedTensor(
            ragged_dims=self.ragged_dims, packed_dim_order=self.packed_dim_order, _sizes=sizes, _concat=values
        )

    def transpose(self, a, b):
        n = self.dim()
        a, b = (x + n if x < 0 else x for x in (a, b))
        if a == 0 or b == 0:
            raise ValueError("the batch axis cannot be transposed")
        a, b = a - 1, b - 1

        def swap(d):
            return b if d == a else a if d == b else d

        sizes = []
        for s in self._sizes:
            s = list(s)
            s[a], s[b] = s[b], s[a]
            sizes.append(tuple(s))
        return NestedTensor(
            ragged_dims=tuple(swap(d) for d in self.ragged_dims),
            packed_dim_order=tuple(swap(d) for d in self.packed_dim_order),
            _sizes=sizes,
            _concat=self.concat,
        )

    def unbind(self):
        out = []
        offsets = self.packed_offsets().tolist()
        order = self.packed_dim_order
        inverse = [order.index(d) for d in range(len(order))]
        for s, lo, hi in zip(self._sizes, offsets[:-1], offsets[1:]):
            block = self.concat[lo:hi].reshape(*(s[d] for d in order))
            out.append(block.permute(inverse))
        return tuple(out)

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        if func is torch.unbind and isinstance(args[0], NestedTensor):
            return args[0].unbind()
        return NotImplemented
