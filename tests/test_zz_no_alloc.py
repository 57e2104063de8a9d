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


def _problem(n, h, c, seed):
    """Starting-node q/k/v (1, n, n, h, c) bf16, row-shared bias (h, n, n), its table and geometry."""

    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(1, n, n, h, c, generator=g).to(torch.bfloat16).to(DEV) for _ in range(3))
    bias = torch.randn(h, n, n, generator=g).to(torch.bfloat16).to(DEV)
    qs = (0, n * h * c, c, h * c)
    table = _core.table_row(groups=n, len_q=n, len_k=n, q=qs, k=qs, v=qs, bias=(0, 0, n * n, n),
                            dbias=(0, 0, n * n, n), bias_mode=_lib.BIAS_SHARED, lse_off=0)  # fmt: skip
    host, dev = _core.device_table(table, q.device)
    geo = _lib.Geometry()
    geo.dtype = geo.bias_dtype = _lib.BF16
    geo.num_heads, geo.head_size, geo.num_samples = h, c, 1
    geo.has_bias, geo.has_mask, geo.vec_ok = 1, 0, 1
    geo.scale = c**-0.5
    geo.table_host, geo.table_device = host.data_ptr(), dev.data_ptr()
    return (q, k, v, bias), geo, (host, dev)


def _outputs(q, n, h):
    return torch.empty_like(q), torch.empty_like(q), torch.empty(n * h * n, device=DEV)


def _ptrs(q, k, v, bias, out, lo, lse):
    return [t.data_ptr() for t in (q, k, v)] + [None, bias.data_ptr()] + [t.data_ptr() for t in (out, lo, lse)]


@pytest.mark.parametrize("order", ["large_then_small"])
def test_forward_noalloc_matches_forward(order):
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    for n, seed in ((384, 1), (96, 2)):
        h, c = 4, 32
        (q, k, v, bias), geo, keep = _problem(n, h, c, seed)
        print(f"noalloc forward n={n} h={h} c={c} seed={seed}", flush=True)
        need = lib.oops_attn_forward_workspace_bytes(ctypes.byref(geo))
        assert 0 < need <= _lib.NOALLOC_SCRATCH_BYTES  # the case uses the scratch
        ref = _outputs(q, n, h)
        ws = torch.empty(need, dtype=torch.uint8, device=DEV)
        rc = lib.oops_attn_forward(ctypes.byref(geo), *_ptrs(q, k, v, bias, *ref), ws.data_ptr(), need, stream)
        assert rc == 0, lib.oops_last_error()
        got = _outputs(q, n, h)
        for t in got:
            t.fill_(float("nan"))
        rc = lib.oops_attn_forward_noalloc(ctypes.byref(geo), *_ptrs(q, k, v, bias, *got), stream)
        assert rc == 0, lib.oops_last_error()
        torch.cuda.synchronize()
        for a, b, name in zip(got, ref, ("out", "out_lo", "lse")):
            assert torch.equal(a, b), name
        del keep
