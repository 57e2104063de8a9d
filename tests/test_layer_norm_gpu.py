"""GPU parity of layer_norm against the float64 oracle (oracle/layer_norm.py).

Follows the reference's layer_norm contract (oops/normalization/layer_norm/
layer_norm.py:30-148): float16 / bfloat16 / float32 activations, widths from 1
to 8192 (odd and non-multiple-of-8 widths take the element path), affine in
the activation dtype, float32 over half, or absent; strided rows; nested
values.  Values and the input gradient are compared elementwise; the affine
gradients (sums over every row) with the tolerance scaled by their largest
magnitude, as the reference's gradient checks do.
"""

import numpy as np
import pytest
import torch

from accuracy import assert_close
from nested_standin import NestedTensor
from oops_amd import LayerNorm, OOpsUnsupportedError, layer_norm
from oracle import layer_norm as oln

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _np(t):
    return None if t is None else t.detach().double().cpu().numpy()


def _grad_close(got, want, dtype, what):
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    err = np.abs(_np(got) - want).max()
    assert err <= tol * max(1.0, float(np.abs(want).max())), f"{what}: {err:.3g}"


# float32 affine over a float32 activation is the "same" case, so it is not listed twice
_CASES = [(d, a) for d in (torch.float32, torch.bfloat16, torch.float16) for a in ("same", "f32", "none")
          if not (a == "f32" and d == torch.float32)]  # fmt: skip


@pytest.mark.parametrize("dtype,affine", _CASES)
@pytest.mark.parametrize("width", [1, 17, 128, 384, 1024, 4096, 8192])
def test_layer_norm(dtype, width, affine):
    g = torch.Generator().manual_seed(width)
    rows = 3000 if width <= 384 else 200
    x = (torch.randn(rows, width, generator=g) * 2 + 0.5).to(dtype).to(DEV).requires_grad_(True)
    wdt = torch.float32 if affine == "f32" else dtype
    w = b = None
    if affine != "none":
        w = torch.randn(width, generator=g).to(wdt).to(DEV).requires_grad_(True)
        b = torch.randn(width, generator=g).to(wdt).to(DEV).requires_grad_(True)
    y = layer_norm(x, width, w, b)
    assert y.shape == x.shape and y.dtype == dtype
    assert_close(y, oln.layer_norm_forward(_np(x), _np(w), _np(b)), dtype, "y")
    dy = torch.randn(rows, width, generator=g).to(dtype).to(DEV)
    leaves = [x] + ([w, b] if w is not None else [])
    got = torch.autograd.grad(y, leaves, dy)
    dx, dw, db = oln.layer_norm_backward(_np(x), _np(dy), _np(w))
    assert_close(got[0], dx, dtype, "dx")
    if w is not None:
        assert got[1].dtype == wdt and got[2].dtype == wdt
        _grad_close(got[1], dw, dtype, "dweight")
        _grad_close(got[2], db, dtype, "dbias")


def test_layer_norm_strided_and_prefix():
    g = torch.Generator().manual_seed(2)
    base = torch.randn(4, 50, 96, generator=g).to(torch.bfloat16).to(DEV)
    x = base[:, :, :64].requires_grad_(False)  # rows 96 elements apart
    w = torch.randn(64, generator=g).to(DEV)
    y = layer_norm(x, (64,), w, None)
    assert_close(y, oln.layer_norm_forward(_np(x), _np(w)), torch.bfloat16, "y")


def test_layer_norm_nested():
    tmpl = NestedTensor([torch.empty(n, 3, 32) for n in (5, 9)], ragged_dims=(0,))
    g = torch.Generator().manual_seed(4)
    vals = torch.randn(tmpl.concat.shape, generator=g).to(torch.bfloat16).to(DEV)
    out = layer_norm(tmpl.packed_like(vals), 32)
    assert isinstance(out, NestedTensor)
    assert_close(out.concat, oln.layer_norm_forward(_np(vals)), torch.bfloat16, "nested")


def test_layer_norm_errors():
    x = torch.randn(4, 8, device=DEV)
    with pytest.raises(OOpsUnsupportedError):
        layer_norm(x, (2, 4))
    with pytest.raises(OOpsUnsupportedError):
        layer_norm(x.double(), 8)
    with pytest.raises(OOpsUnsupportedError):
        layer_norm(x, 8, torch.ones(8, device=DEV, dtype=torch.bfloat16))  # half affine over float32
    with pytest.raises(OOpsUnsupportedError):
        layer_norm(torch.randn(4, 9000, device=DEV), 9000)


def test_layer_norm_compile_matches_eager():
    g = torch.Generator().manual_seed(8)
    x0 = torch.randn(64, 96, generator=g).to(torch.bfloat16).to(DEV)
    w = torch.randn(96, generator=g).to(DEV).requires_grad_(True)
    dy = torch.randn(64, 96, generator=g).to(torch.bfloat16).to(DEV)

    def run(x):
        return layer_norm(x, 96, w, None)

    results = []
    for fn in (run, torch.compile(run, fullgraph=True)):
        x = x0.clone().requires_grad_(True)
        y = fn(x)
        results.append((y.detach(), *torch.autograd.grad(y, [x, w], dy)))
    for got, ref in zip(*results):
        torch.testing.assert_close(got, ref, atol=0, rtol=0)


def test_layer_norm_module():
    """oops_amd.LayerNorm (reference oops/normalization/layer_norm/modules.py:31-70): torch.nn.LayerNorm's
    constructor and parameters; CUDA half/float32 calls run the HIP kernels, declined inputs (float64,
    several normalized dimensions) fall back to PyTorch's LayerNorm."""

    import importlib

    ln_mod = importlib.import_module("oops_amd.normalization.layer_norm")

    torch.manual_seed(3)
    m = LayerNorm(96, eps=1e-6).to(DEV)
    assert isinstance(m, torch.nn.LayerNorm)
    with torch.no_grad():
        m.weight.normal_()
        m.bias.normal_()
    x = torch.randn(4, 50, 96, device=DEV).to(torch.bfloat16).requires_grad_(True)
    calls = []
    real = ln_mod._apply
    ln_mod._apply = lambda *a: calls.append(1) or real(*a)
    try:
        y = m(x)
    finally:
        ln_mod._apply = real
    assert calls, "the module did not run the HIP path"
    assert_close(y, oln.layer_norm_forward(_np(x), _np(m.weight), _np(m.bias), eps=1e-6), torch.bfloat16, "y")
    dy = torch.randn_like(y)
    gx, gw, gb = torch.autograd.grad(y, (x, m.weight, m.bias), dy)
    dx, dw, db = oln.layer_norm_backward(_np(x), _np(dy), _np(m.weight), eps=1e-6)
    assert_close(gx, dx, torch.bfloat16, "dx")
    _grad_close(gw, dw, torch.bfloat16, "dweight")
    _grad_close(gb, db, torch.bfloat16, "dbias")
    # declined by layer_norm -> native LayerNorm
    m64 = LayerNorm(96).to(DEV).double()
    x64 = torch.randn(3, 96, device=DEV, dtype=torch.float64)
    torch.testing.assert_close(m64(x64), torch.nn.functional.layer_norm(x64, (96,), m64.weight, m64.bias))
    m2 = LayerNorm((5, 96)).to(DEV)
    x2 = torch.randn(2, 5, 96, device=DEV)
    torch.testing.assert_close(m2(x2), torch.nn.functional.layer_norm(x2, (5, 96), m2.weight, m2.bias))


def test_layer_norm_backward_affine_abi():
    """oops_layer_norm_rows_backward_affine: the backward with the affine gradients summed in the library.
    dx equals the partial-writing entry point's bit for bit; the sums equal a float64 sum of its partials,
    and repeated calls are bit-identical (fixed summation order, two launches of chunk sums here)."""

    import ctypes
    import importlib

    from oops_amd import _lib

    ln = importlib.import_module("oops_amd.normalization.layer_norm")
    lib = _lib.load()
    rows, width = 1 << 17, 128
    g = torch.Generator().manual_seed(21)
    x = torch.randn(rows, width, generator=g).to(torch.bfloat16).to(DEV)
    w = torch.randn(width, generator=g).to(DEV)
    dy = torch.randn(rows, width, generator=g).to(torch.bfloat16).to(DEV)
    _, mean, rstd = ln.layer_norm_forward(x, w, None, 1e-5)
    geo = ln._geometry(x.dtype, rows, width, width, 1e-5)
    parts = lib.oops_layer_norm_rows_parts(ctypes.byref(geo))
    assert parts > 256, "the chunked (two-launch) sum is the case under test"
    stream = torch.cuda.current_stream().cuda_stream
    acc = torch.empty(2, parts, width, device=DEV)
    dx_ref = torch.empty_like(x)
    rc = lib.oops_layer_norm_rows_backward(ctypes.byref(geo), x.data_ptr(), w.data_ptr(), mean.data_ptr(),
                                           rstd.data_ptr(), dy.data_ptr(), dx_ref.data_ptr(), acc[0].data_ptr(),
                                           acc[1].data_ptr(), stream)  # fmt: skip
    assert rc == 0, lib.oops_last_error()
    need = lib.oops_layer_norm_rows_backward_workspace_bytes(ctypes.byref(geo))
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    outs = []
    for _ in range(2):
        dx = torch.full_like(x, float("nan"))
        dw, db = torch.full((width,), float("nan"), device=DEV), torch.full((width,), float("nan"), device=DEV)
        rc = lib.oops_layer_norm_rows_backward_affine(ctypes.byref(geo), x.data_ptr(), w.data_ptr(), mean.data_ptr(),
                                                      rstd.data_ptr(), dy.data_ptr(), dx.data_ptr(), dw.data_ptr(),
                                                      db.data_ptr(), ws.data_ptr(), need, stream)  # fmt: skip
        assert rc == 0, lib.oops_last_error()
        outs.append((dx, dw, db))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], dx_ref)
    want = acc.double().sum(1)
    for got, ref, name in ((outs[0][1], want[0], "dweight"), (outs[0][2], want[1], "dbias")):
        err = (got.double() - ref).abs().max().item()
        assert err <= 1e-5 * max(1.0, ref.abs().max().item()), f"{name}: {err:.3g}"
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a, b)
