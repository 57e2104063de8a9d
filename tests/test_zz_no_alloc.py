"""oops_attn_forward_noalloc: the forward entry point that allocates nothing.

It runs the kernels of oops_attn_forward with the fragment-major bias copy in
the library's static device scratch instead of a caller workspace, so its
results must equal oops_attn_forward's bit for bit.  Two calls in a row (the
second on a smaller problem, which reuses the scratch the first one filled)
are each compared with oops_attn_forward on the same inputs, through the C ABI.
This entry point has no counterpart in the reference.
"""

import ctypes

import pytest
import torch

from oops_amd import _lib
from oops_amd.attention import _core

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _problem(n, h, c, seed, dtype=torch.bfloat16, masked=False):
    """Starting-node q/k/v (1, n, n, h, c), row-shared bias (h, n, n), an optional key mask (n, n) with
    masked and mixed 64-key tiles, the table and the geometry."""

    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(1, n, n, h, c, generator=g).to(dtype).to(DEV) for _ in range(3))
    bias = torch.randn(h, n, n, generator=g).to(dtype).to(DEV)
    mask = None
    if masked:
        keep = torch.rand(n, n, generator=g) > 0.2
        keep[:, 0] = True
        keep[1, 64:128] = False  # a fully masked tile
        mask = keep.to(torch.uint8).to(DEV)
    qs = (0, n * h * c, c, h * c)
    table = _core.table_row(groups=n, len_q=n, len_k=n, q=qs, k=qs, v=qs, bias=(0, 0, n * n, n),
                            dbias=(0, 0, n * n, n), bias_mode=_lib.BIAS_SHARED,
                            mask=None if mask is None else (0, n, 0), lse_off=0)  # fmt: skip
    host, dev = _core.device_table(table, q.device)
    geo = _lib.Geometry()
    geo.dtype = geo.bias_dtype = _lib.BF16 if dtype == torch.bfloat16 else _lib.F16
    geo.num_heads, geo.head_size, geo.num_samples = h, c, 1
    geo.has_bias, geo.has_mask, geo.vec_ok = 1, int(masked), 1
    geo.scale = c**-0.5
    geo.table_host, geo.table_device = host.data_ptr(), dev.data_ptr()
    return (q, k, v, mask, bias), geo, (host, dev)


def _msa_problem(s_, h, n, c, seed):
    """Head-major MSA rows q/k/v (s_, h, n, c) bf16 with a row-shared bias (h, n, n) whose
    fragment-major copy exceeds the no-allocation scratch."""

    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(s_, h, n, c, generator=g).to(torch.bfloat16).to(DEV) for _ in range(3))
    bias = torch.randn(h, n, n, generator=g).to(torch.bfloat16).to(DEV)
    qs = (0, h * n * c, n * c, c)
    table = _core.table_row(groups=s_, len_q=n, len_k=n, q=qs, k=qs, v=qs, bias=(0, 0, n * n, n),
                            dbias=(0, 0, n * n, n), bias_mode=_lib.BIAS_SHARED, lse_off=0)  # fmt: skip
    host, dev = _core.device_table(table, q.device)
    geo = _lib.Geometry()
    geo.dtype = geo.bias_dtype = _lib.BF16
    geo.num_heads, geo.head_size, geo.num_samples = h, c, 1
    geo.has_bias, geo.has_mask, geo.vec_ok = 1, 0, 1
    geo.scale = c**-0.5
    geo.table_host, geo.table_device = host.data_ptr(), dev.data_ptr()
    return (q, k, v, None, bias), geo, (host, dev)


def _outputs(q, rows):
    return torch.empty_like(q), torch.empty_like(q), torch.empty(rows, device=DEV)


def _ptrs(q, k, v, mask, bias, out, lo, lse):
    return [t.data_ptr() for t in (q, k, v)] + [None if mask is None else mask.data_ptr(), bias.data_ptr()] + [
        t.data_ptr() for t in (out, lo, lse)
    ]


def _compare(lib, tensors, geo, lse_rows, within_scratch):
    """oops_attn_forward_noalloc against oops_attn_forward (caller workspace) on the same inputs."""

    stream = torch.cuda.current_stream().cuda_stream
    q = tensors[0]
    need = lib.oops_attn_forward_workspace_bytes(ctypes.byref(geo))
    assert need > 0
    assert (need <= _lib.NOALLOC_SCRATCH_BYTES) == within_scratch
    ref = _outputs(q, lse_rows)
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    rc = lib.oops_attn_forward(ctypes.byref(geo), *_ptrs(*tensors, *ref), ws.data_ptr(), need, stream)
    assert rc == 0, lib.oops_last_error()
    got = _outputs(q, lse_rows)
    for t in got:
        t.fill_(float("nan"))
    rc = lib.oops_attn_forward_noalloc(ctypes.byref(geo), *_ptrs(*tensors, *got), stream)
    assert rc == 0, lib.oops_last_error()
    torch.cuda.synchronize()
    for a, b, name in zip(got, ref, ("out", "out_lo", "lse")):
        assert torch.equal(a, b), name


@pytest.mark.parametrize(
    "dtype,masked", [(torch.bfloat16, False), (torch.bfloat16, True), (torch.float16, True)]
)  # fmt: skip
def test_forward_noalloc_matches_forward(dtype, masked):
    """Two calls in a row, the second smaller (it reuses the scratch the first one filled)."""

    lib = _lib.load()
    for n, seed in ((384, 1), (96, 2)):
        h, c = 4, 32
        tensors, geo, keep = _problem(n, h, c, seed, dtype, masked)
        print(f"noalloc forward n={n} h={h} c={c} seed={seed} {dtype} masked={masked}", flush=True)
        _compare(lib, tensors, geo, n * h * n, True)
        del keep


def test_forward_noalloc_beyond_scratch():
    """A bias whose fragment-major copy (35.7 MB) exceeds the 32 MiB scratch: the no-allocation forward
    reads the bias rows directly instead, with the same results as the forward that copies them."""

    lib = _lib.load()
    s_, h, n, c = 2, 16, 1056, 32
    tensors, geo, keep = _msa_problem(s_, h, n, c, 5)
    print(f"noalloc forward beyond the scratch: S={s_} H={h} N={n} c={c}", flush=True)
    _compare(lib, tensors, geo, s_ * h * n, False)
    del keep
