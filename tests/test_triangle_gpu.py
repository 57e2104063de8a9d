"""GPU parity of dense triangle attention against the numpy oracle.

Cases follow the reference's test matrix (tests/attention/triangle/
test_triangle_attention.py:226-419): dtypes, starting/ending-node
("swapped") layouts, prefix axes, shared/full/no bias, fp32 bias over half
inputs, masks, odd head sizes, neg-bit views and aliasing.  Tolerances are
those of BASELINE.json, read as max-abs error divided by max(1, |ref|)
(absolute for unit-scale values, relative for larger ones, whose 16-bit
output rounding alone would exceed 2e-2): fp32 <= 1e-5; 16-bit <= 2e-2 and
mean-relative <= 1e-2, against the float64 oracle on the same (rounded)
inputs.
"""

import numpy as np
import pytest
import torch

from oracle import attention as ora
from oops_amd import OOpsUnsupportedError, triangle_attention
from oops_amd.attention import _core

from accuracy import assert_close

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _np(t):
    return None if t is None else t.detach().double().cpu().numpy()


def make_case(dtype, *, prefix=(2,), rows=4, cols=33, heads=2, head=24, bias_kind="shared", masked=True,
              layout="dense", bias_dtype=None, seed=0):
    g = torch.Generator().manual_seed(seed)
    shape = (*prefix, rows, cols, heads, head)
    if layout == "swapped":
        base = [torch.randn((*prefix, cols, rows, heads, head), generator=g).to(dtype) for _ in range(3)]
        q, k, v = (b.transpose(-4, -3) for b in base)
    else:
        q, k, v = (torch.randn(shape, generator=g).to(dtype) for _ in range(3))
    mask = None
    if masked:
        mask = torch.rand((*prefix, rows, cols), generator=g) > 0.2
        mask[..., 0] = True
    bias = None
    if bias_kind != "none":
        bshape = (*prefix, 1 if bias_kind == "shared" else rows, heads, cols, cols)
        bias = torch.randn(bshape, generator=g).to(bias_dtype or dtype)
    dout = torch.randn(shape, generator=g).to(dtype)
    return q, k, v, mask, bias, dout


def run_and_check(q, k, v, mask, bias, dout, dtype, grads=True, scale=None, grad_tol16=2e-2):
    to = lambda t: None if t is None else t.to(DEV)
    leaves = []
    dq, dk, dv, db = (to(t) for t in (q, k, v, bias))
    if q.dim() >= 5 and not q.is_contiguous():  # keep the swapped layout on device
        dq, dk, dv = (torch.empty_strided(t.shape, t.stride(), dtype=t.dtype, device=DEV).copy_(t) for t in (q, k, v))
    tensors = []
    for t in (dq, dk, dv, db):
        if t is not None and grads:
            t.requires_grad_(True)
            leaves.append(t)
        tensors.append(t)
    out = triangle_attention(tensors[0], tensors[1], tensors[2], to(mask), tensors[3], scale=scale)
    assert out.shape == q.shape and out.dtype == q.dtype
    m = _np(mask)
    exp_out, _ = ora.triangle_attention_forward(_np(q), _np(k), _np(v), m, _np(bias), scale)
    assert_close(out, exp_out, dtype, "out")
    if not grads:
        return
    got = torch.autograd.grad(out, leaves, to(dout))
    want = ora.triangle_attention_backward(_np(q), _np(k), _np(v), _np(dout), m, _np(bias), scale)
    names = ("dq", "dk", "dv", "dbias")
    for g_, w, leaf, name in zip(got, want, leaves, names):
        assert g_.dtype == leaf.dtype and g_.shape == leaf.shape
        assert_close(g_, w, dtype, name, tol16=grad_tol16)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bias_kind", ["none", "shared", "full"])
@pytest.mark.parametrize("layout", ["dense", "swapped"])
def test_forward_backward(dtype, bias_kind, layout):
    case = make_case(dtype, bias_kind=bias_kind, layout=layout)
    run_and_check(*case, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("masked", [False, True])
@pytest.mark.parametrize("cols", [33, 64, 130])
def test_generic_kernels_match_oracle(dtype, masked, cols):
    """The generic (non-fast-path) kernels on 16-bit inputs, forced."""

    case = make_case(dtype, cols=cols, head=32, masked=masked, seed=cols)
    with _core.force_generic():
        run_and_check(*case, dtype)


@pytest.mark.parametrize("cols", [1, 7, 64, 65, 200])
@pytest.mark.parametrize("head", [8, 32, 48, 64])
def test_fast_path_shapes(cols, head):
    case = make_case(torch.bfloat16, rows=3, cols=cols, head=head, seed=head + cols)
    run_and_check(*case, torch.bfloat16)


def test_fast_path_masked_tiles():
    """Fully kept, fully masked and mixed 64-key tiles in one row set."""

    q, k, v, mask, bias, dout = make_case(torch.bfloat16, rows=4, cols=256, head=32, seed=21)
    mask[:] = True
    mask[0, 0, 64:128] = False  # a fully masked tile
    mask[0, 1, 5] = False  # a mixed tile
    mask[0, 2, :] = False  # a fully masked row
    mask[1, 3, 200:] = False  # tail
    run_and_check(q, k, v, mask, bias, dout, torch.bfloat16)


def test_large_logits_lazy_rescale():
    """Growing logits along the key axis exercise the lazy max update."""

    q, k, v, mask, bias, dout = make_case(torch.bfloat16, rows=2, cols=320, head=32, bias_kind="shared", seed=4)
    ramp = torch.linspace(-40, 40, 320)
    bias = (bias.float() + ramp).to(torch.bfloat16)
    # gradients: the reference's own bf16 tolerance (test_triangle_attention.py:35-39); with
    # P ~ 1 on the same keys for every query, rounding P to bf16 before the dV
    # product (as the reference does) alone costs ~1.7% here
    run_and_check(q, k, v, None, bias, dout, torch.bfloat16, grad_tol16=5e-2)


@pytest.mark.parametrize("head", [16, 32, 64, 128, 129, 255])
def test_head_sizes_fp32(head):
    case = make_case(torch.float32, rows=3, cols=17, head=head, seed=117)
    run_and_check(*case, torch.float32)


@pytest.mark.parametrize("head", [16, 24, 32, 64, 128, 129])
def test_head_sizes_bf16(head):
    case = make_case(torch.bfloat16, rows=3, cols=41, head=head, seed=3)
    run_and_check(*case, torch.bfloat16)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fp32_bias_over_half(dtype):
    case = make_case(dtype, bias_kind="full", bias_dtype=torch.float32)
    run_and_check(*case, dtype)


def test_prefixed_and_batchless():
    case = make_case(torch.float32, prefix=(2, 3), rows=3, cols=19, head=16)
    run_and_check(*case, torch.float32)
    case = make_case(torch.float32, prefix=(), rows=5, cols=37, head=32, bias_kind="none")
    q, k, v, mask, bias, dout = case
    run_and_check(q, k, v, mask, None, dout, torch.float32)


def test_scale_and_long_rows():
    case = make_case(torch.bfloat16, prefix=(1,), rows=3, cols=300, heads=4, head=32, seed=5)
    run_and_check(*case, torch.bfloat16, scale=0.3)


def test_negative_view_and_alias():
    q, k, v, mask, bias, dout = make_case(torch.float32, cols=21, head=16)
    qd = q.to(DEV).requires_grad_(True)
    out = triangle_attention(torch._neg_view(qd), torch._neg_view(qd), torch._neg_view(qd), mask.to(DEV))
    exp, _ = ora.triangle_attention_forward(-_np(q), -_np(q), -_np(q), _np(mask))
    assert_close(out, exp, torch.float32, "neg out")
    (gq,) = torch.autograd.grad(out, (qd,), dout.to(DEV))
    want = ora.triangle_attention_backward(-_np(q), -_np(q), -_np(q), _np(dout), _np(mask))
    assert_close(gq, -(want[0] + want[1] + want[2]), torch.float32, "alias grad")


def test_fully_masked_nonfinite():
    q, k, v = (torch.full((1, 17, 17, 2, 129), float("inf"), device=DEV, requires_grad=True) for _ in range(3))
    mask = torch.zeros(1, 17, 17, device=DEV, dtype=torch.bool)
    bias = torch.full((1, 1, 2, 17, 17), float("nan"), device=DEV, requires_grad=True)
    out = triangle_attention(q, k, v, mask, bias)
    torch.testing.assert_close(out, torch.zeros_like(out))
    for grad, leaf in zip(torch.autograd.grad(out.sum(), (q, k, v, bias)), (q, k, v, bias)):
        torch.testing.assert_close(grad, torch.zeros_like(leaf))


@pytest.mark.parametrize("cols,rows", [(200, 3), (900, 2)])
def test_masked_keys_nonfinite_fast_path(cols, rows):
    """bf16 fast path with a shared bias and mixed 64-key tiles (the key mask folded into the bias fragments,
    the fused dK/dV + dBias kernel with two or eight waves per row): inf in the K rows and NaN in the V rows
    of masked keys, and NaN in the bias column of a key masked in every row, change no output and no
    gradient against the same call with finite values there."""

    q, k, v, mask, bias, dout = make_case(torch.bfloat16, prefix=(1,), rows=rows, cols=cols, heads=4, head=32,
                                          seed=cols)  # fmt: skip
    kc = cols // 3
    mask[..., kc] = False  # masked in every row: its bias column may hold anything
    q, k, v, bias, dout, mask = (t.to(DEV) for t in (q, k, v, bias, dout, mask))

    def run(k_, v_, b_):
        leaves = [t.detach().clone().requires_grad_(True) for t in (q, k_, v_, b_)]
        out = triangle_attention(leaves[0], leaves[1], leaves[2], mask, leaves[3])
        return (out, *torch.autograd.grad(out, leaves, dout))

    clean = run(k, v, bias)
    off = ~mask  # (1, rows, cols): masked (row, key) pairs
    kp, vp, bp = k.clone(), v.clone(), bias.clone()
    kp[off] = float("inf")
    vp[off] = float("nan")
    bp[..., kc] = float("nan")
    poisoned = run(kp, vp, bp)
    for name, a_, b_ in zip(("out", "dq", "dk", "dv", "dbias"), clean, poisoned):
        if name == "dbias":
            a_, b_ = a_[..., torch.arange(cols) != kc], b_[..., torch.arange(cols) != kc]
        elif name in ("dk", "dv"):
            a_, b_ = a_[mask], b_[mask]
        assert torch.isfinite(b_).all(), name
        assert torch.equal(a_, b_), name


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bias_kind", ["shared", "full"])
def test_additive_neg_inf_bias(dtype, bias_kind):
    """-inf in the bias works as an additive key mask on the 16-bit fast paths: the bias passes through an
    identity MFMA there, so a non-finite element must not turn the 16 keys it is summed with into NaN.
    Every output and gradient is finite and matches the call that masks the same key through ``mask``."""

    cols, kc = 200, 7
    q, k, v, _, bias, dout = make_case(dtype, prefix=(1,), rows=3, cols=cols, heads=4, head=32, masked=False,
                                       bias_kind=bias_kind, seed=3)  # fmt: skip
    q, k, v, bias, dout = (t.to(DEV) for t in (q, k, v, bias, dout))
    b_inf, b_zero = bias.clone(), bias.clone()
    b_inf[..., kc] = float("-inf")
    b_zero[..., kc] = 0
    mask = torch.ones(1, 3, cols, dtype=torch.bool, device=DEV)
    mask[..., kc] = False

    def run(b_, m_):
        leaves = [t.detach().clone().requires_grad_(True) for t in (q, k, v, b_)]
        out = triangle_attention(leaves[0], leaves[1], leaves[2], m_, leaves[3])
        return (out, *torch.autograd.grad(out, leaves, dout))

    additive, masked = run(b_inf, None), run(b_zero, mask)
    for name, a_, b_ in zip(("out", "dq", "dk", "dv", "dbias"), additive, masked):
        assert torch.isfinite(a_).all(), name
        torch.testing.assert_close(a_.float(), b_.float(), atol=2e-2, rtol=2e-2, msg=name)


def test_rows_fully_masked_partially():
    q, k, v, mask, bias, dout = make_case(torch.bfloat16, rows=6, cols=40, head=32, seed=9)
    mask[:, 2] = False
    run_and_check(q, k, v, mask, bias, dout, torch.bfloat16)


def test_config_c2_key_padding():
    """BASELINE config 2 at full size: N=384, H=4, c=32, bf16, last 10-30% keys padded (seed 1)."""

    torch.manual_seed(1)
    n, h, c = 384, 4, 32
    q, k, v, dout = (torch.randn(1, n, n, h, c).to(torch.bfloat16) for _ in range(4))
    bias = torch.randn(1, 1, h, n, n).to(torch.bfloat16)
    frac = float(torch.empty(1).uniform_(0.10, 0.30, generator=torch.Generator().manual_seed(1)))
    keep_len = n - round(n * frac)
    mask = torch.ones(1, n, n, dtype=torch.bool)
    mask[..., keep_len:] = False
    mask[:, keep_len:, :] = False
    run_and_check(q, k, v, mask, bias, dout, torch.bfloat16)


def test_errors():
    q = torch.randn(1, 3, 5, 2, 8, device=DEV)
    with pytest.raises(ValueError):
        triangle_attention(q, q, q[..., :-1])
    with pytest.raises(OOpsUnsupportedError):
        triangle_attention(q.double(), q.double(), q.double())
    with pytest.raises(OOpsUnsupportedError):
        triangle_attention(q, q, q, torch.ones(1, 3, 5, device=DEV))  # non-bool mask


def test_unmasked_swapped_fast_path():
    """Ending-node layout without a mask: the unmasked-tile (MASKED_TILES=false) fast kernels."""

    for bias_kind in ("shared", "full", "none"):
        case = make_case(torch.bfloat16, rows=5, cols=192, heads=4, head=32, bias_kind=bias_kind, masked=False,
                         layout="swapped", seed=31)  # fmt: skip
        run_and_check(*case, torch.bfloat16)


def test_config_c1_fp32():
    """starting node, fp32, N=64, H=4, c=32, no mask, forward and gradients
    against the full float64 oracle at 1e-5 (tests/attention/triangle/test_triangle_attention.py:42-63)."""

    g = torch.Generator().manual_seed(1)
    n, h, c = 64, 4, 32
    q, k, v, dout = (torch.randn(1, n, n, h, c, generator=g) for _ in range(4))
    bias = torch.randn(1, 1, h, n, n, generator=g)
    run_and_check(q, k, v, None, bias, dout, torch.float32)


def _report(name, got, want):
    got = got.detach().double().cpu().numpy()
    err = np.abs(got - want)
    print(f"c3 {name}: max-abs {err.max():.3g} mean-rel {err.mean() / max(np.abs(want).mean(), 1e-30):.3g}", flush=True)


def test_config_c3_ending_node():
    """BASELINE config 3 (the headline) at full size, on exactly the benchmark's inputs
    (bench.make_inputs: seed 2, randn(1,768,768,4,32) bf16 passed as .transpose(1,2) views, shared
    bias (1,1,4,768,768), no mask, upstream gradient in the output's layout).

    Rows are independent, so O, dQ, dK and dV are checked against the float64 oracle on 4 rows.
    The shared dBias sums dS over all 768 rows; it is checked against the float64 oracle over every
    row on 6 query positions (all heads, all keys), through the oracle's pair-bias form, whose
    queries may be a subset of the keys.
    """

    from bench import make_inputs, step

    q, k, v, bias, dout = make_inputs(DEV)
    out = triangle_attention(q, k, v, None, bias)
    dq, dk, dv, db = torch.autograd.grad(out, (q, k, v, bias), dout)
    # the benchmark's own step returns the same gradients (no state between calls)
    for a_, b_ in zip(step(q, k, v, bias, dout), (dq, dk, dv, db)):
        assert torch.equal(a_, b_)
    qn, kn, vn, don, bn = (_np(t) for t in (q, k, v, dout, bias))
    rows = [0, 257, 511, 767]
    exp_out, _ = ora.triangle_attention_forward(qn[:, rows], kn[:, rows], vn[:, rows], None, bn)
    want = ora.triangle_attention_backward(qn[:, rows], kn[:, rows], vn[:, rows], don[:, rows], None, bn)
    for name, got, w in zip(("out", "dq", "dk", "dv"), (out, dq, dk, dv), (exp_out, *want[:3])):
        _report(name, got[:, rows], w)
        assert_close(got[:, rows], w, torch.bfloat16, name)
    # dBias over every row, head-major (S=rows, H, Q, D) pair-bias form restricted to a query subset
    # (exact: queries are independent): 6 positions for every head, and for head 0 a 1-in-8 stride over
    # all 768 queries whose offset within each block of 8 rotates, so every 32-query tile (one wave-step
    # of the fused kernel) and every position of the accumulator layout is checked
    hm = lambda x: np.swapaxes(x[0], 1, 2)  # (rows, cols, H, D) -> (rows, H, cols, D)
    qh, kh, vh, dh = (hm(x.astype(np.float32)) for x in (qn, kn, vn, don))
    qpos = [0, 1, 100, 383, 640, 767]
    strided = [8 * j + (3 * j) % 8 for j in range(96)]
    with _core.capture_dbias_f32() as cap:
        out2 = triangle_attention(q, k, v, None, bias)
        (db2,) = torch.autograd.grad(out2, (bias,), dout)
    assert torch.equal(db2, db)
    db32 = cap.values[0][0, 0]
    for name, heads, pos in (("dbias", slice(None), qpos), ("dbias head 0 strided", slice(0, 1), strided)):
        want_db = ora.shared_dbias_at(qh[:, heads], kh[:, heads], vh[:, heads], dh[:, heads], None,
                                      bn[0, :, heads], pos)  # fmt: skip
        _report(name, db[0, 0][heads][:, pos], want_db)
        assert_close(db[0, 0][heads][:, pos], want_db, torch.bfloat16, name)
        # the float32 sums before the cast to bf16 meet 2e-2 max-abs outright
        err32 = np.abs(_np(db32[heads][:, pos]) - want_db).max()
        print(f"c3 {name} float32 before the cast: max-abs {err32:.3g}", flush=True)
        assert err32 <= 2e-2, (name, err32)


@pytest.mark.parametrize(
    "cols,rows,masked,layout",
    [(96, 5, True, "swapped"), (200, 3, True, "dense"), (40, 4, False, "swapped"), (768, 2, False, "swapped"),
     (33, 6, True, "dense"), (384, 64, True, "dense"), (1024, 3, True, "dense"), (800, 2, False, "swapped"),
     (1000, 5, True, "swapped"), (300, 7, True, "swapped"), (160, 9, False, "dense"), (384, 5, False, "swapped")],
)  # fmt: skip
def test_fused_dkv_dbias(cols, rows, masked, layout):
    """The fused dK/dV + shared-dBias kernel (16-bit, head size <= 32, row-shared bias; two waves per row
    from 129 to 384 queries, four up to 768, eight up to 1024; rows not a multiple of the rows in flight):
    oracle parity, agreement with the separate dK/dV and dBias kernels, and bit-identical repeats."""

    case = make_case(torch.bfloat16, prefix=(1,), rows=rows, cols=cols, heads=4, head=32, masked=masked,
                     layout=layout, seed=cols + rows)  # fmt: skip
    run_and_check(*case, torch.bfloat16)
    q, k, v, mask, bias, dout = (None if t is None else t.to(DEV) for t in case)
    if layout == "swapped":
        q, k, v = (torch.empty_strided(t.shape, t.stride(), dtype=t.dtype, device=DEV).copy_(t) for t in (q, k, v))

    def grads():
        leaves = [t.detach().clone().requires_grad_(True) for t in (q, k, v, bias)]
        out = triangle_attention(leaves[0], leaves[1], leaves[2], mask, leaves[3])
        return torch.autograd.grad(out, leaves, dout)

    fused = grads()
    again = grads()
    for a_, b_ in zip(fused, again):
        assert torch.equal(a_, b_)
    with _core.separate_dkv_dbias():
        separate = grads()
    for name, a_, b_ in zip(("dq", "dk", "dv", "dbias"), fused, separate):
        err = (a_.float() - b_.float()).abs().max().item()
        assert err <= 2e-2 * max(1.0, b_.float().abs().max().item()), (name, err)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_large_bias_nondefault_scale(dtype):
    """The fast kernels add the bias through an identity MFMA whose weight 1/scale is rounded to the
    input dtype: the bias term is scaled by 1 + d with |d| <= 2^-9 (bf16) or 2^-11 (f16), a logit shift of
    at most |d| |bias|.  With scale 0.3 (bf16 rounds 1/0.3 by 0.1%) and biases of magnitude ~30 the shift
    reaches ~0.03; the outputs and gradients still meet the 16-bit tolerance against the float64 oracle."""

    q, k, v, mask, bias, dout = make_case(dtype, prefix=(1,), rows=3, cols=96, heads=2, head=32, masked=False,
                                          layout="swapped", seed=21)  # fmt: skip
    bias = (bias.float() * 30.0).to(dtype)
    run_and_check(q, k, v, mask, bias, dout, dtype, scale=0.3)
