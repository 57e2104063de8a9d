"""oops_sum_partials on the GPU: the fixed summation order restated in float32 numpy is matched bit for bit,
and the rounding to a 16-bit output is the round-to-nearest-even of that float32 sum."""

import ctypes

import numpy as np
import pytest
import torch

from oops_amd import _lib
from oops_amd._partials import PartialSums

pytestmark = pytest.mark.gpu
DEV = "cuda"


def quarter_sum(rows: np.ndarray) -> np.ndarray:
    """float32 sum of up to 256 rows in the kernel's order: slice s sums the s-th quarter of the rows in
    order (quarters of ceil(rows / 4)), then (s0 + s1) + (s2 + s3)."""

    count, n = rows.shape
    q = (count + 3) // 4
    sl = []
    for s in range(4):
        acc = np.zeros(n, np.float32)
        for p in range(s * q, min(count, (s + 1) * q)):
            acc = (acc + rows[p]).astype(np.float32)
        sl.append(acc)
    return ((sl[0] + sl[1]).astype(np.float32) + (sl[2] + sl[3]).astype(np.float32)).astype(np.float32)


def fixed_order_sum(parts: np.ndarray) -> np.ndarray:
    """Up to 256 rows: one quarter_sum; more: quarter_sum of each 256-row chunk, then of the chunk sums."""

    if parts.shape[0] <= 256:
        return quarter_sum(parts)
    chunks = np.stack([quarter_sum(parts[c : c + 256]) for c in range(0, parts.shape[0], 256)])
    return quarter_sum(chunks)


@pytest.mark.parametrize(
    "count,n", [(0, 7), (1, 5), (5, 64), (7, 1000), (64, 65536 * 2 + 3), (65, 33), (256, 40), (257, 33), (2048, 70),
                (8193, 130)]
)
def test_sum_partials_matches_the_fixed_order(count, n):
    g = torch.Generator().manual_seed(count * 7 + n)
    parts = torch.randn(count, n, generator=g) * 10
    sums = PartialSums()
    out = sums.add(parts.to(DEV))
    sums.run(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), fixed_order_sum(parts.numpy()))


def test_sum_partials_strided_rows_16bit_outputs_and_many_segments():
    """Rows spaced wider than n, bf16 / f16 results, and more arrays than one launch takes."""

    g = torch.Generator().manual_seed(3)
    base = torch.randn(9, 40, generator=g)
    strided = base.to(DEV)[:, :33]  # part_stride 40 > n 33
    arrays = [torch.randn(3 + i, 17 + 5 * i, generator=g) for i in range(_lib.SUM_MAX_SEGMENTS + 3)]
    sums = PartialSums()
    o_strided = sums.add(strided, torch.bfloat16)
    outs = [sums.add(a.to(DEV), torch.float16 if i % 2 else torch.float32) for i, a in enumerate(arrays)]
    sums.run(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    ref = torch.from_numpy(fixed_order_sum(base[:, :33].numpy()))
    assert torch.equal(o_strided.cpu(), ref.to(torch.bfloat16))
    for i, (a, o) in enumerate(zip(arrays, outs)):
        ref = torch.from_numpy(fixed_order_sum(a.numpy()))
        assert torch.equal(o.cpu(), ref.to(o.dtype)), i


def test_sum_partials_is_bit_identical_across_calls():
    g = torch.Generator().manual_seed(5)
    parts = (torch.randn(300, 4097, generator=g) * 100).to(DEV)
    res = []
    for _ in range(3):
        sums = PartialSums()
        res.append(sums.add(parts))
        sums.run(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(res[0], res[1]) and torch.equal(res[1], res[2])


def test_sum_partials_through_the_c_abi_reports_launch_errors_cleanly():
    lib = _lib.load()
    x = torch.ones(4, 8, device=DEV)
    out = torch.empty(8, device=DEV)
    seg = (_lib.SumSegment * 1)()
    seg[0].parts, seg[0].out, seg[0].count, seg[0].n, seg[0].part_stride = x.data_ptr(), out.data_ptr(), 4, 8, 8
    seg[0].out_dtype = _lib.F32
    assert lib.oops_sum_partials(seg, 1, None, 0, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) == 0
    torch.cuda.synchronize()
    assert torch.equal(out, torch.full((8,), 4.0, device=DEV))
