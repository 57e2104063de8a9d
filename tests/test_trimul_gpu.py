"""GPU parity of triangle_multiplication against the float64 oracle (oracle/trimul.py).

Mirrors the reference's cases (tests/pair/triangle_multiplication/
test_triangle_multiplication.py:305-330): odd channel and hidden widths
(C = 17, 65, H = 12, 24, 96), both directions, with and without projection
biases, float and bool masks, prefixes, strided and broadcast masks, nested
ragged pairs with and without a static prefix, and an AlphaFold-sized
C = H = 128 pair.  Forward values use the oracle with the reference's
storage roundings; gradients (pair, mask, every weight and bias) are checked
against the oracle's float64 derivative with the reference's gradient
criterion (error within tol x the gradient tensor's largest magnitude).
"""

import numpy as np
import pytest
import torch

from accuracy import assert_close
from nested_standin import NestedTensor
from oops_amd import OOpsUnsupportedError, triangle_multiplication
from oracle import trimul as otm

pytestmark = pytest.mark.gpu

DEV = "cuda"
_ROUNDING = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: None}
_NAMES = ("input_norm_weight", "input_norm_bias", "left_value_weight", "left_gate_weight", "right_value_weight",
          "right_gate_weight", "output_norm_weight", "output_norm_bias", "output_weight", "output_gate_weight")
_BIAS = ("left_value_bias", "left_gate_bias", "right_value_bias", "right_gate_bias", "output_bias",
         "output_gate_bias")  # fmt: skip


# the reference's gradient criterion for this operator
# (tests/pair/triangle_multiplication/test_triangle_multiplication.py:36-40, :458-464):
# |got - want| <= tol * max(1, max |want|) over each gradient tensor
_GRAD_TOL = {torch.bfloat16: 5e-2, torch.float16: 3e-2, torch.float32: 1e-5}


def _assert_grad_close(got, want, dtype, what):
    got = got.detach().double().cpu().numpy()
    err = np.abs(got - want).max()
    scale = max(1.0, float(np.abs(want).max()))
    assert err <= _GRAD_TOL[dtype] * scale, f"{what}: max-abs {err:.3g} against {_GRAD_TOL[dtype]} x {scale:.3g}"


def _np(t):
    return None if t is None else t.detach().double().cpu().numpy()


def _params(dtype, c, h, seed, biases=True, norm_dtype=None):
    g = torch.Generator().manual_seed(seed)
    nd = norm_dtype or dtype

    def r(*shape, scale=1.0, dt=dtype):
        return (torch.randn(*shape, generator=g) * scale).to(dt).to(DEV).requires_grad_(True)

    weights = (r(c, dt=nd), r(c, dt=nd), r(h, c, scale=c**-0.5), r(h, c, scale=c**-0.5), r(h, c, scale=c**-0.5),
               r(h, c, scale=c**-0.5), r(h, dt=nd), r(h, dt=nd), r(c, h, scale=h**-0.5), r(c, c, scale=c**-0.5))  # fmt: skip
    bs = tuple(r(w, scale=0.2) for w in (h, h, h, h, c, c)) if biases else (None,) * 6
    return weights, bs


def _call(pair, mask, weights, bs, direction):
    kw = dict(zip(_NAMES, weights))
    kw.update({k: v for k, v in zip(_BIAS, bs)})
    return triangle_multiplication(pair, mask, direction=direction, **kw)


def _check(pair, mask, weights, bs, direction, dtype, grads=True, mask_grad=False):
    out = _call(pair, mask, weights, bs, direction)
    assert out.shape == pair.shape and out.dtype == dtype
    np_w, np_b = [_np(w) for w in weights], [_np(b) for b in bs]
    want = otm.triangle_multiplication_forward(_np(pair), _np(mask), np_w, np_b, direction,
                                               rounding=_ROUNDING[dtype])  # fmt: skip
    assert_close(out, want, dtype, "out")
    if not grads:
        return
    dy = torch.randn(out.shape, generator=torch.Generator().manual_seed(11)).to(dtype).to(DEV)
    leaves = [pair, *weights, *[b for b in bs if b is not None]] + ([mask] if mask_grad else [])
    got = torch.autograd.grad(out, leaves, dy)
    d_pair, d_mask, d_w, d_b = otm.triangle_multiplication_backward(_np(pair), _np(mask), np_w, np_b, _np(dy),
                                                                    direction)  # fmt: skip
    want_g = [d_pair, *d_w, *[b for b in d_b if b is not None]] + ([d_mask] if mask_grad else [])
    names = ["pair", *_NAMES, *[n for n, b in zip(_BIAS, bs) if b is not None]] + (["mask"] if mask_grad else [])
    for name, g_, w_ in zip(names, got, want_g):
        assert g_.shape == tuple(w_.shape), name
        _assert_grad_close(g_, w_, dtype, "d" + name)


@pytest.mark.parametrize(
    "dtype,c,h,n,prefix,direction,biases",
    [
        (torch.bfloat16, 32, 32, 16, (2,), "outgoing", True),
        (torch.bfloat16, 32, 32, 16, (2,), "incoming", True),
        (torch.bfloat16, 32, 32, 12, (), "incoming", True),  # 4 | positions, 16 does not: 8-byte factor stores
        (torch.float16, 64, 64, 48, (), "outgoing", True),  # 16 | positions: traded 32-byte stores
        (torch.bfloat16, 32, 96, 48, (), "incoming", True),  # 16 | positions, the second channel block partial
        (torch.float16, 128, 64, 32, (3,), "outgoing", True),  # 16 | positions, several tiles per workgroup
        (torch.bfloat16, 192, 64, 16, (2,), "outgoing", True),  # three k panels, run as four (the last zero)
        (torch.float16, 256, 32, 32, (), "incoming", False),  # four k panels, no mask
        (torch.float16, 8, 12, 9, (), "outgoing", False),
        (torch.bfloat16, 17, 24, 7, (), "outgoing", True),
        (torch.float16, 65, 96, 17, (), "incoming", True),
        (torch.bfloat16, 128, 128, 19, (2, 3), "outgoing", False),
        (torch.bfloat16, 128, 128, 64, (1,), "incoming", True),
        (torch.bfloat16, 384, 384, 33, (), "outgoing", False),  # c_row > 256: W streamed through LDS
        (torch.float16, 1024, 8, 5, (), "incoming", True),  # widest pair, narrow hidden
        (torch.bfloat16, 8, 1024, 5, (), "outgoing", True),  # widest hidden (few positions per LDS tile)
        (torch.float32, 17, 24, 7, (2,), "outgoing", True),
        (torch.float32, 8, 12, 9, (), "incoming", False),
        (torch.float32, 128, 128, 20, (1,), "incoming", True),  # 4 | positions: float4 factor stores
        (torch.float32, 65, 96, 17, (), "outgoing", True),  # odd widths, two channel blocks of W
        (torch.float32, 40, 200, 12, (), "outgoing", False),  # four hidden blocks, the last partial
    ],
)
def test_trimul_dense(dtype, c, h, n, prefix, direction, biases):
    g = torch.Generator().manual_seed(c + h + n)
    pair = torch.randn(*prefix, n, n, c, generator=g).to(dtype).to(DEV).requires_grad_(True)
    mask = (torch.rand(*prefix, n, n, generator=g) > 0.2).to(DEV)
    weights, bs = _params(dtype, c, h, seed=n, biases=biases)
    _check(pair, mask, weights, bs, direction, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_trimul_float_mask_gradient_and_broadcast(dtype):
    """A fractional float mask broadcast over the prefix: its gradient is summed over the prefix."""

    g = torch.Generator().manual_seed(4)
    pair = torch.randn(3, 12, 12, 32, generator=g).to(dtype).to(DEV).requires_grad_(True)
    mask = torch.rand(1, 12, 12, generator=g).to(DEV).requires_grad_(True)
    weights, bs = _params(dtype, 32, 48, seed=5)
    _check(pair, mask, weights, bs, "incoming", dtype, mask_grad=True)


def test_trimul_float32_runs_the_fused_kernels(monkeypatch):
    """float32 pairs go through the same fused implementation as 16-bit ones (the float32 MFMA kernels of
    csrc/trimul_f32.hip), not a composition of library ops."""

    import importlib

    mod = importlib.import_module("oops_amd.pair.triangle_multiplication")
    calls = []
    orig = mod._forward_impl
    monkeypatch.setattr(mod, "_forward_impl", lambda *a: calls.append(a[0].dtype) or orig(*a))
    dtype = torch.float32
    g = torch.Generator().manual_seed(9)
    pair = torch.randn(2, 9, 9, 24, generator=g).to(DEV).requires_grad_(True)
    mask = (torch.rand(2, 9, 9, generator=g) > 0.3).to(DEV)
    weights, bs = _params(dtype, 24, 40, seed=9)
    _check(pair, mask, weights, bs, "outgoing", dtype)
    assert calls == [torch.float32]


def test_trimul_no_mask_fp32_norm_weights():
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(6)
    pair = torch.randn(2, 10, 10, 24, generator=g).to(dtype).to(DEV).requires_grad_(True)
    weights, bs = _params(dtype, 24, 40, seed=6, norm_dtype=torch.float32)
    _check(pair, None, weights, bs, "outgoing", dtype)


def test_trimul_strided_pair():
    """A non-contiguous pair view (the reference's 'strided' layout)."""

    dtype = torch.float16
    g = torch.Generator().manual_seed(8)
    base = torch.randn(11, 11, 40, 2, generator=g).to(dtype).to(DEV)
    pair = base[..., 0].requires_grad_(False)
    assert not pair.is_contiguous()
    weights, bs = _params(dtype, 40, 32, seed=8)
    out = _call(pair, None, weights, bs, "outgoing")
    want = otm.triangle_multiplication_forward(_np(pair), None, [_np(w) for w in weights], [_np(b) for b in bs],
                                               "outgoing", rounding="f16")  # fmt: skip
    assert_close(out, want, dtype, "out")


@pytest.mark.parametrize("prefix,direction", [((), "outgoing"), ((2,), "incoming")])
def test_trimul_nested(prefix, direction):
    dtype = torch.bfloat16
    lengths = (5, 12, 9)
    c, h = 32, 48
    pr = len(prefix)
    tmpl = NestedTensor([torch.empty(*prefix, n, n, c) for n in lengths], ragged_dims=(pr, pr + 1))
    g = torch.Generator().manual_seed(3)
    values = torch.randn(tmpl.concat.shape, generator=g).to(dtype).to(DEV).requires_grad_(True)
    pair = tmpl.packed_like(values)
    mtmpl = NestedTensor([torch.empty(*prefix, n, n) for n in lengths], ragged_dims=(pr, pr + 1))
    mask = mtmpl.packed_like((torch.rand(mtmpl.concat.shape, generator=g) > 0.2).float().to(DEV))
    weights, bs = _params(dtype, c, h, seed=3)
    out = _call(pair, mask, weights, bs, direction)
    assert isinstance(out, NestedTensor) and out.concat.shape == values.shape
    dy = torch.randn(values.shape, generator=g).to(dtype).to(DEV)
    got = torch.autograd.grad(out.concat, [values, weights[2], weights[8]], dy)
    np_w, np_b = [_np(w) for w in weights], [_np(b) for b in bs]
    d_pairs, d_wlv, d_wo = [], 0.0, 0.0
    dys = out.packed_like(dy).unbind()
    for i, (pe, me, oe, de) in enumerate(zip(pair.unbind(), mask.unbind(), out.unbind(), dys)):
        want = otm.triangle_multiplication_forward(_np(pe), _np(me), np_w, np_b, direction, rounding="bf16")
        assert_close(oe, want, dtype, f"out[{i}]")
        dp, _, dw, _ = otm.triangle_multiplication_backward(_np(pe), _np(me), np_w, np_b, _np(de), direction)
        d_pairs.append(torch.from_numpy(dp))
        d_wlv, d_wo = d_wlv + dw[2], d_wo + dw[8]
    _assert_grad_close(got[0], torch.cat([pair._pack(d) for d in d_pairs]).numpy(), dtype, "dpair")
    _assert_grad_close(got[1], d_wlv, dtype, "d_left_value_weight")
    _assert_grad_close(got[2], d_wo, dtype, "d_output_weight")


def test_trimul_alphafold_size():
    """N = 256, C = H = 128, bf16: forward against the oracle on the full pair; gradients of the pair
    and the output projection against the oracle."""

    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(12)
    n = 256
    pair = torch.randn(n, n, 128, generator=g).to(dtype).to(DEV).requires_grad_(True)
    mask = (torch.rand(n, n, generator=g) > 0.1).to(DEV)
    weights, bs = _params(dtype, 128, 128, seed=12)
    _check(pair, mask, weights, bs, "outgoing", dtype)


def test_trimul_errors():
    weights, bs = _params(torch.bfloat16, 16, 8, seed=1)
    pair = torch.randn(4, 4, 16, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        _call(pair, None, weights, bs, "sideways")
    with pytest.raises(ValueError):
        _call(pair[:, :3], None, weights, bs, "outgoing")
    with pytest.raises(ValueError):
        _call(pair, torch.ones(5, 4, device=DEV), weights, bs, "outgoing")
    with pytest.raises(ValueError):
        _call(pair, None, (weights[0][:-1], *weights[1:]), bs, "outgoing")
    fw, fb = _params(torch.float64, 16, 8, seed=1)  # float64 is not served
    with pytest.raises(OOpsUnsupportedError):
        _call(pair.double(), None, fw, fb, "outgoing")


def test_trimul_compile_matches_eager():
    """torch.compile(fullgraph=True) traces the custom ops (the reference tests its compile mode)."""

    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(21)
    pair0 = torch.randn(2, 12, 12, 32, generator=g).to(dtype).to(DEV)
    mask = (torch.rand(2, 12, 12, generator=g) > 0.2).float().to(DEV)
    weights, bs = _params(dtype, 32, 48, seed=21)
    dy = torch.randn(2, 12, 12, 32, generator=g).to(dtype).to(DEV)

    def run(p):
        return _call(p, mask, weights, bs, "incoming")

    results = []
    for fn in (run, torch.compile(run, fullgraph=True)):
        p = pair0.clone().requires_grad_(True)
        out = fn(p)
        results.append((out.detach(), *torch.autograd.grad(out, [p, weights[2], bs[0]], dy)))
    for got, ref in zip(*results):
        torch.testing.assert_close(got, ref, atol=0, rtol=0)


@pytest.mark.parametrize("dtype,groups,positions", [(torch.float16, 3, 173), (torch.bfloat16, 1, 128), (torch.bfloat16, 7, 4097)])
def test_trimul_output_grad_products(dtype, groups, positions):
    """oops_trimul_output_grad_products through the C-ABI against float64 products of the same 16-bit inputs:
    D = X W rounded once to 16 bits, the per-workgroup partials of X^T Y and of X's column sums summed in
    float64.  Ragged row counts (not a multiple of the 128-row tile) and padded row strides."""

    import ctypes

    from oops_amd import _lib

    lib = _lib.load()
    R, C = groups * positions, 128
    g = torch.Generator().manual_seed(positions)
    x = torch.randn(R, C + 8, generator=g).to(dtype).to(DEV)[:, :C]
    y = torch.randn(R, C + 16, generator=g).to(dtype).to(DEV)[:, 8:8 + C]
    w = (torch.randn(C, C, generator=g) * C**-0.5).to(dtype).to(DEV)
    d = torch.full((R, C + 8), 7.0, dtype=dtype, device=DEV)
    geo = _lib.TrimulGeometry()
    geo.dtype = _lib.BF16 if dtype == torch.bfloat16 else _lib.F16
    geo.channels, geo.hidden, geo.has_mask = C, C, 0
    geo.groups, geo.positions, geo.c_row, geo.h_row, geo.eps = groups, positions, C, C, 1e-5
    parts = lib.oops_trimul_output_grad_parts(ctypes.byref(geo))
    assert parts >= 1
    gp = torch.full((parts, C, C), float("nan"), device=DEV)
    sp = torch.full((parts, C), float("nan"), device=DEV)
    rc = lib.oops_trimul_output_grad_products(ctypes.byref(geo), x.data_ptr(), x.stride(0), w.data_ptr(), C,
                                              y.data_ptr(), y.stride(0), d.data_ptr(), d.stride(0), gp.data_ptr(),
                                              sp.data_ptr(), torch.cuda.current_stream().cuda_stream)  # fmt: skip
    assert rc == 0, lib.oops_last_error()
    torch.cuda.synchronize()
    xd, yd, wd = x.double().cpu(), y.double().cpu(), w.double().cpu()
    want_d = (xd @ wd).to(dtype).double()
    got_d = d[:, :C].double().cpu()
    # one rounding of a float32 accumulation: within an ulp of the 16-bit result
    ulp = 2.0 ** (-7 if dtype == torch.bfloat16 else -10)
    assert ((got_d - want_d).abs() <= ulp * want_d.abs().clamp_min(2.0**-6) + 1e-6).all()
    assert (d[:, C:] == 7.0).all()  # the padding past each row stays untouched
    got_g, got_s = gp.double().sum(0).cpu(), sp.double().sum(0).cpu()
    want_g, want_s = xd.t() @ yd, xd.sum(0)
    assert (got_g - want_g).abs().max().item() <= 1e-5 * max(1.0, want_g.abs().max().item()) * (R**0.5)
    assert (got_s - want_s).abs().max().item() <= 1e-5 * max(1.0, want_s.abs().max().item()) * (R**0.5)
