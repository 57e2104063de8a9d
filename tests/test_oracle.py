"""Pins the numpy oracle (oracle/attention.py) against independent routes.

* torch.nn.functional.scaled_dot_product_attention (library routine), forward
  and autograd, with the bias passed as a float attn_mask (so dBias is pinned);
* a pure-Python brute-force loop (index / transposition mistakes);
* central finite differences of the oracle forward (the analytic backward);
* invariants: ending node == starting node on transposed tensors, shared
  dBias == row-sum of full dBias, probabilities sum to one, fully masked rows
  give zero output and zero gradients even with non-finite inputs.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as ora


def _rand(rng, *shape):
    return rng.standard_normal(shape)


def _sdpa_triangle(q, k, v, mask, bias, scale):
    """Triangle attention through SDPA on (B, R, H, C, D) tensors; float attn_mask carries bias and mask."""

    qt, kt, vt = (x.transpose(-2, -3) for x in (q, k, v))
    B, R, H, C, D = qt.shape
    attn = torch.zeros(B, R, H, C, C, dtype=q.dtype)
    if bias is not None:
        attn = attn + bias
    if mask is not None:
        attn = attn.masked_fill(~mask[:, :, None, None, :], float("-inf"))
    out = F.scaled_dot_product_attention(qt, kt, vt, attn_mask=attn, scale=scale)
    return out.transpose(-2, -3)


@pytest.mark.parametrize("bias_kind", ["none", "shared", "full"])
@pytest.mark.parametrize("masked", [False, True])
def test_forward_backward_vs_sdpa(bias_kind, masked):
    rng = np.random.default_rng(7)
    B, R, C, H, D = 2, 5, 9, 3, 8
    q, k, v, do = (_rand(rng, B, R, C, H, D) for _ in range(4))
    bias = None if bias_kind == "none" else _rand(rng, B, 1 if bias_kind == "shared" else R, H, C, C)
    mask = None
    if masked:
        mask = rng.random((B, R, C)) > 0.3
        mask[..., 0] = True  # SDPA returns NaN on fully masked rows; those are pinned separately
    scale = 0.37
    out, _ = ora.triangle_attention_forward(q, k, v, mask, bias, scale)
    dq, dk, dv, db = ora.triangle_attention_backward(q, k, v, do, mask, bias, scale)

    tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    tb = None if bias is None else torch.tensor(bias, requires_grad=True)
    tm = None if mask is None else torch.tensor(mask)
    ref = _sdpa_triangle(tq, tk, tv, tm, tb, scale)
    np.testing.assert_allclose(out, ref.detach().numpy(), atol=1e-12, rtol=1e-10)
    leaves = [tq, tk, tv] + ([tb] if tb is not None else [])
    grads = torch.autograd.grad(ref, leaves, torch.tensor(do))
    for mine, theirs in zip((dq, dk, dv, db), grads):
        np.testing.assert_allclose(mine, theirs.numpy(), atol=1e-11, rtol=1e-9)


def test_bruteforce_loops():
    rng = np.random.default_rng(3)
    q, k, v = (_rand(rng, 1, 3, 4, 2, 3) for _ in range(3))
    bias = _rand(rng, 1, 3, 2, 4, 4)
    mask = np.array([[[1, 0, 1, 1], [0, 0, 0, 0], [1, 1, 0, 1]]], dtype=bool)
    out, _ = ora.triangle_attention_forward(q, k, v, mask, bias)
    brute = ora.triangle_attention_bruteforce(q, k, v, mask, bias)
    np.testing.assert_allclose(out, brute, atol=1e-13)
    assert np.all(out[0, 1] == 0.0)  # row 1 has no kept key


def test_finite_differences():
    rng = np.random.default_rng(11)
    q, k, v, do = (_rand(rng, 1, 2, 4, 2, 3) for _ in range(4))
    bias = _rand(rng, 1, 1, 2, 4, 4)
    mask = np.array([[[1, 1, 0, 1], [1, 0, 1, 1]]], dtype=bool)
    grads = ora.triangle_attention_backward(q, k, v, do, mask, bias)
    args = [q, k, v, bias]
    eps = 1e-6
    for idx, g in enumerate(grads):
        x = args[idx]
        num = np.zeros_like(x)
        it = np.nditer(x, flags=["multi_index"])
        for _ in it:
            i = it.multi_index
            saved = x[i]
            x[i] = saved + eps
            fp = (ora.triangle_attention_forward(*args[:3], mask, args[3])[0] * do).sum()
            x[i] = saved - eps
            fm = (ora.triangle_attention_forward(*args[:3], mask, args[3])[0] * do).sum()
            x[i] = saved
            num[i] = (fp - fm) / (2 * eps)
        np.testing.assert_allclose(g, num, atol=1e-7, rtol=1e-6)


def test_invariants():
    rng = np.random.default_rng(5)
    B, R, C, H, D = 1, 4, 6, 2, 5
    q, k, v, do = (_rand(rng, B, R, C, H, D) for _ in range(4))
    # ending node == starting node on swapped pair axes
    out, _ = ora.triangle_attention_forward(q, k, v)
    sw = [np.swapaxes(x, 1, 2) for x in (q, k, v)]
    out_sw, _ = ora.triangle_attention_forward(*sw)
    direct = ora.triangle_attention_bruteforce(*sw)
    np.testing.assert_allclose(out_sw, direct, atol=1e-12)
    assert not np.allclose(out, np.swapaxes(out_sw, 1, 2))  # orientation matters
    # shared-bias gradient == sum over rows of the full-bias gradient
    shared = _rand(rng, B, 1, H, C, C)
    full = np.broadcast_to(shared, (B, R, H, C, C)).copy()
    db_shared = ora.triangle_attention_backward(q, k, v, do, None, shared)[3]
    db_full = ora.triangle_attention_backward(q, k, v, do, None, full)[3]
    np.testing.assert_allclose(db_shared, db_full.sum(axis=1, keepdims=True), atol=1e-12)
    # a bias broadcast over the prefix: its gradient is the prefix sum of the expanded bias's
    q2, k2, v2, do2 = (_rand(rng, 2, R, C, H, D) for _ in range(4))
    bb = _rand(rng, 1, 1, H, C, C)
    db_b = ora.triangle_attention_backward(q2, k2, v2, do2, None, bb)[3]
    db_e = ora.triangle_attention_backward(q2, k2, v2, do2, None, np.broadcast_to(bb, (2, 1, H, C, C)).copy())[3]
    assert db_b.shape == bb.shape
    np.testing.assert_allclose(db_b, db_e.sum(axis=0, keepdims=True), atol=1e-12)
    # dV == P^T dO with P rows summing to 1
    s = np.einsum("brihd,brjhd->brhij", q, k) * D**-0.5
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    np.testing.assert_allclose(p.sum(-1), 1.0, atol=1e-12)
    dv = ora.triangle_attention_backward(q, k, v, do)[2]
    np.testing.assert_allclose(dv, np.einsum("brhij,brihd->brjhd", p, do), atol=1e-12)
    # LSE == logsumexp of the scores
    _, lse = ora.triangle_attention_forward(q, k, v)
    np.testing.assert_allclose(lse, np.log(np.exp(s).sum(-1)), atol=1e-12)


def test_fully_masked_nonfinite():
    q = np.full((1, 3, 3, 1, 4), np.inf)
    bias = np.full((1, 1, 1, 3, 3), np.nan)
    mask = np.zeros((1, 3, 3), dtype=bool)
    with np.errstate(invalid="ignore"):
        out, lse = ora.triangle_attention_forward(q, q, q, mask, bias)
        grads = ora.triangle_attention_backward(q, q, q, np.ones_like(q), mask, bias)
    assert np.all(out == 0) and np.all(lse == 0)
    for g in grads:
        assert np.all(g == 0)


@pytest.mark.parametrize("mask_kind", ["none", "key", "pair"])
def test_pair_bias_vs_sdpa(mask_kind):
    rng = np.random.default_rng(13)
    S, H, Q, D = 3, 2, 7, 4
    q, k, v, do = (_rand(rng, S, H, Q, D) for _ in range(4))
    bias = _rand(rng, 1, H, Q, Q)
    mask = None
    if mask_kind == "key":
        mask = rng.random((S, Q)) > 0.3
        mask[:, 0] = True
    elif mask_kind == "pair":
        mask = rng.random((S, Q, Q)) > 0.3
        mask[..., 0] = True
    out = ora.pair_bias_attention_forward(q, k, v, mask, bias)
    grads = ora.pair_bias_attention_backward(q, k, v, do, mask, bias)
    tq, tk, tv, tb = (torch.tensor(x, requires_grad=True) for x in (q, k, v, bias))
    attn = tb.expand(S, H, Q, Q)
    if mask is not None:
        keep = torch.tensor(mask)
        keep = keep[:, None, None, :] if mask_kind == "key" else keep[:, None]
        attn = attn.masked_fill(~keep, float("-inf"))
    ref = F.scaled_dot_product_attention(tq, tk, tv, attn_mask=attn)
    np.testing.assert_allclose(out, ref.detach().numpy(), atol=1e-12)
    tgrads = torch.autograd.grad(ref, (tq, tk, tv, tb), torch.tensor(do))
    for mine, theirs in zip(grads, tgrads):
        np.testing.assert_allclose(mine, theirs.numpy(), atol=1e-11)


def test_shared_dbias_at_vs_sdpa():
    """The chunked query-subset dBias the full-size GPU tests use equals SDPA autograd's bias gradient
    (bias broadcast over the rows, key mask) restricted to those queries."""

    rng = np.random.default_rng(17)
    S, H, Q, D = 9, 2, 12, 4
    q, k, v, do = (_rand(rng, S, H, Q, D) for _ in range(4))
    bias = _rand(rng, 1, H, Q, Q)
    mask = rng.random((S, Q)) > 0.3
    mask[:, 0] = True
    qpos = [0, 5, 11, 7]
    got = ora.shared_dbias_at(q, k, v, do, mask, bias, qpos, rows_per_chunk=4)
    tq, tk, tv, tb = (torch.tensor(x, requires_grad=True) for x in (q, k, v, bias))
    attn = tb.expand(S, H, Q, Q).masked_fill(~torch.tensor(mask)[:, None, None, :], float("-inf"))
    ref = F.scaled_dot_product_attention(tq, tk, tv, attn_mask=attn)
    (tgb,) = torch.autograd.grad(ref, (tb,), torch.tensor(do))
    np.testing.assert_allclose(got, tgb.numpy()[0][:, qpos], atol=1e-11)


# ------------------------------------------------------------------ gate oracle


def test_gate_docstring_example():
    """The reference's own example (gate_attention_output.py:73-81): zero gate logits halve the values."""

    from oracle import gate as gora

    out, _, _ = gora.gate_attention_output_forward(np.ones((1, 1, 2)), np.zeros((1, 3)), np.zeros((2, 3)), np.ones((1, 2)))
    assert out.tolist() == [[1.0]]


def test_gate_vs_torch_autograd():
    """Forward and all four gradients against torch autograd of the composition (float64)."""

    from oracle import gate as gora

    g = torch.Generator().manual_seed(0)
    att = torch.randn(2, 3, 4, 5, 8, generator=g, dtype=torch.float64, requires_grad=True)  # (B, S, H, Q, D)
    single = torch.randn(2, 3, 5, 7, generator=g, dtype=torch.float64, requires_grad=True)
    w = torch.randn(32, 7, generator=g, dtype=torch.float64, requires_grad=True)
    wo = torch.randn(6, 32, generator=g, dtype=torch.float64, requires_grad=True)
    flat = att.transpose(-3, -2).reshape(2, 3, 5, 32)
    out = F.linear(torch.sigmoid(F.linear(single, w)) * flat, wo)
    dy = torch.randn(out.shape, generator=g, dtype=torch.float64)
    want = torch.autograd.grad(out, (att, single, w, wo), dy)
    got_out, _, _ = gora.gate_attention_output_forward(att.detach().numpy(), single.detach().numpy(),
                                                       w.detach().numpy(), wo.detach().numpy())
    np.testing.assert_allclose(got_out, out.detach().numpy(), rtol=1e-12, atol=1e-12)
    got = gora.gate_attention_output_backward(att.detach().numpy(), single.detach().numpy(), w.detach().numpy(),
                                              wo.detach().numpy(), dy.numpy())
    for a, b in zip(got, want):
        np.testing.assert_allclose(a, b.numpy(), rtol=1e-10, atol=1e-10)


def test_gate_finite_differences():
    """The written-out derivative against central differences of the forward."""

    from oracle import gate as gora

    rng = np.random.default_rng(1)
    att = rng.standard_normal((2, 3, 4))  # (H, Q, D)
    single = rng.standard_normal((3, 5))
    w = rng.standard_normal((8, 5))
    wo = rng.standard_normal((2, 8))
    dy = rng.standard_normal((3, 2))
    grads = gora.gate_attention_output_backward(att, single, w, wo, dy)
    eps = 1e-6
    for i, x in enumerate((att, single, w, wo)):
        fd = np.zeros_like(x)
        for idx in np.ndindex(x.shape):
            xp, xm = x.copy(), x.copy()
            xp[idx] += eps
            xm[idx] -= eps
            args_p = [att, single, w, wo]
            args_m = [att, single, w, wo]
            args_p[i], args_m[i] = xp, xm
            fp = (gora.gate_attention_output_forward(*args_p)[0] * dy).sum()
            fm = (gora.gate_attention_output_forward(*args_m)[0] * dy).sum()
            fd[idx] = (fp - fm) / (2 * eps)
        np.testing.assert_allclose(grads[i], fd, rtol=1e-5, atol=1e-6)


def test_gate_rounding_points_vs_torch_bf16():
    """With bf16 rounding the oracle's stored intermediates equal torch's bf16 composition."""

    from oracle import gate as gora

    g = torch.Generator().manual_seed(2)
    att = torch.randn(3, 4, 9, 16, generator=g).to(torch.bfloat16)
    single = torch.randn(3, 9, 24, generator=g).to(torch.bfloat16)
    w = torch.randn(64, 24, generator=g).to(torch.bfloat16)
    wo = torch.randn(8, 64, generator=g).to(torch.bfloat16)
    logits = torch.nn.functional.linear(single.float(), w.float()).to(torch.bfloat16)
    gate = torch.sigmoid(logits.float()).to(torch.bfloat16)
    gated = (gate.float() * att.transpose(-3, -2).reshape(3, 9, 64).float()).to(torch.bfloat16)
    _, got_gated, got_logits = gora.gate_attention_output_forward(
        att.double().numpy(), single.double().numpy(), w.double().numpy(), wo.double().numpy(), rounding="bf16")
    np.testing.assert_array_equal(got_logits, logits.double().numpy())
    np.testing.assert_array_equal(got_gated, gated.double().numpy())


# ------------------------------------------------------------------ triangle multiplicative update

from oracle import trimul as otm  # noqa: E402


def _trimul_case(seed, n=5, c=6, h=4, prefix=(2,), biases=True):
    g = np.random.default_rng(seed)
    pair = g.standard_normal((*prefix, n, n, c))
    mask = (g.random((*prefix, n, n)) > 0.2).astype(np.float64) * g.uniform(0.5, 1.5, (*prefix, n, n))
    weights = (
        g.standard_normal(c), g.standard_normal(c),
        g.standard_normal((h, c)) / c**0.5, g.standard_normal((h, c)) / c**0.5,
        g.standard_normal((h, c)) / c**0.5, g.standard_normal((h, c)) / c**0.5,
        g.standard_normal(h), g.standard_normal(h),
        g.standard_normal((c, h)) / h**0.5, g.standard_normal((c, c)) / c**0.5,
    )  # fmt: skip
    bs = tuple(0.2 * g.standard_normal(w) for w in (h, h, h, h, c, c)) if biases else (None,) * 6
    return pair, mask, weights, bs


def _trimul_torch(pair, mask, weights, biases, direction):
    """The reference test's own formulation (test_triangle_multiplication.py:166-198) in torch."""

    iw, ib, wlv, wlg, wrv, wrg, ow, ob, wo, wog = weights
    blv, blg, brv, brg, bo, bog = biases
    normalized = F.layer_norm(pair, (pair.shape[-1],), iw, ib, 1e-5)
    left = F.linear(normalized, wlv, blv) * torch.sigmoid(F.linear(normalized, wlg, blg))
    right = F.linear(normalized, wrv, brv) * torch.sigmoid(F.linear(normalized, wrg, brg))
    if mask is not None:
        left = left * mask.unsqueeze(-1)
        right = right * mask.unsqueeze(-1)
    left, right = left.movedim(-1, -3), right.movedim(-1, -3)
    combined = left @ right.transpose(-1, -2) if direction == "outgoing" else left.transpose(-1, -2) @ right
    combined = combined.movedim(-3, -1)
    update = F.layer_norm(combined, (combined.shape[-1],), ow, ob, 1e-5)
    return F.linear(update, wo, bo) * torch.sigmoid(F.linear(normalized, wog, bog))


def test_trimul_docstring_example():
    """oops/pair/triangle_multiplication/triangle_multiplication.py:128-145: a constant pair with identity
    weights and zero biases normalizes to zero, so every factor and the update are zero."""

    c = 16
    eye, ones, zeros = np.eye(c), np.ones(c), np.zeros(c)
    weights = (ones, zeros, eye, eye, eye, eye, ones, zeros, eye, eye)
    out = otm.triangle_multiplication_forward(np.ones((2, 2, c)), None, weights)
    assert out.shape == (2, 2, c)
    np.testing.assert_array_equal(out, np.zeros((2, 2, c)))


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
@pytest.mark.parametrize("biases", [True, False])
def test_trimul_vs_torch_autograd(direction, biases):
    pair, mask, weights, bs = _trimul_case(3 + biases, biases=biases)
    want_out = otm.triangle_multiplication_forward(pair, mask, weights, bs, direction)
    t = lambda x: None if x is None else torch.tensor(x, dtype=torch.float64, requires_grad=True)  # noqa: E731
    tp, tm = t(pair), t(mask)
    tw, tb = [t(w) for w in weights], [t(b) for b in bs]
    out = _trimul_torch(tp, tm, tw, tb, direction)
    np.testing.assert_allclose(out.detach().numpy(), want_out, rtol=1e-10, atol=1e-12)
    dy = np.random.default_rng(9).standard_normal(out.shape)
    leaves = [tp, tm, *tw, *[b for b in tb if b is not None]]
    grads = torch.autograd.grad(out, leaves, torch.tensor(dy))
    d_pair, d_mask, d_w, d_b = otm.triangle_multiplication_backward(pair, mask, weights, bs, dy, direction)
    mine = [d_pair, d_mask, *d_w, *[b for b in d_b if b is not None]]
    assert len(mine) == len(grads)
    for got, ref in zip(mine, grads):
        np.testing.assert_allclose(got, ref.numpy(), rtol=1e-9, atol=1e-10)


def test_trimul_broadcast_mask_gradient():
    """A mask broadcast over the prefix gets the prefix-summed gradient."""

    pair, mask, weights, bs = _trimul_case(5, prefix=(3,))
    mask1 = mask[:1]
    dy = np.random.default_rng(2).standard_normal(pair.shape)
    _, d_m, _, _ = otm.triangle_multiplication_backward(pair, mask1, weights, bs, dy)
    _, d_full, _, _ = otm.triangle_multiplication_backward(pair, np.broadcast_to(mask1, mask.shape), weights, bs, dy)
    assert d_m.shape == mask1.shape
    np.testing.assert_allclose(d_m, d_full.sum(0, keepdims=True), rtol=1e-12)


def test_trimul_finite_differences():
    pair, mask, weights, bs = _trimul_case(7, n=4, c=5, h=3, prefix=())
    dy = np.random.default_rng(1).standard_normal(pair.shape)
    d_pair, d_mask, d_w, d_b = otm.triangle_multiplication_backward(pair, mask, weights, bs, dy, "incoming")

    def f(p=pair, m=mask, w=weights, b=bs):
        return (otm.triangle_multiplication_forward(p, m, w, b, "incoming") * dy).sum()

    eps = 1e-6
    rng = np.random.default_rng(0)
    checks = [("pair", pair, d_pair, lambda x: f(p=x)), ("mask", mask, d_mask, lambda x: f(m=x))]
    for i in (0, 2, 7, 9):
        checks.append((f"w{i}", weights[i], d_w[i],
                       lambda x, i=i: f(w=tuple(x if j == i else w for j, w in enumerate(weights)))))  # fmt: skip
    checks.append(("b_og", bs[5], d_b[5], lambda x: f(b=(*bs[:5], x))))
    for name, x0, grad, fn in checks:
        for _ in range(3):
            idx = tuple(rng.integers(0, s) for s in x0.shape)
            xp, xm = x0.copy(), x0.copy()
            xp[idx] += eps
            xm[idx] -= eps
            fd = (fn(xp) - fn(xm)) / (2 * eps)
            assert abs(fd - grad[idx]) < 1e-5 * max(1.0, abs(fd)), (name, idx, fd, grad[idx])


# ------------------------------------------------------------------ layer_norm

from oracle import layer_norm as oln  # noqa: E402


@pytest.mark.parametrize("width", [1, 7, 64])
def test_layer_norm_vs_torch(width):
    g = np.random.default_rng(width)
    x = g.standard_normal((3, 5, width)) * 3 + 1
    w, b, dy = g.standard_normal(width), g.standard_normal(width), g.standard_normal((3, 5, width))
    tx, tw, tb = (torch.tensor(a, requires_grad=True) for a in (x, w, b))
    out = F.layer_norm(tx, (width,), tw, tb, 1e-5)
    np.testing.assert_allclose(oln.layer_norm_forward(x, w, b), out.detach().numpy(), rtol=1e-12, atol=1e-12)
    got = oln.layer_norm_backward(x, dy, w)
    for mine, ref in zip(got, torch.autograd.grad(out, (tx, tw, tb), torch.tensor(dy))):
        np.testing.assert_allclose(mine, ref.numpy(), rtol=1e-10, atol=1e-10)
