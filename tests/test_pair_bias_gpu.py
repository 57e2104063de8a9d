"""GPU parity of dense pair-bias (MSA row) attention against the numpy oracle.

Cases follow the reference's test matrix (tests/attention/pair_bias/
test_pair_bias_attention.py:330-640): dense, negative-view, sliced and
sampled (rank-5) layouts; key, pair and absent masks; full, shared and absent
bias; rectangular query/key lengths; a subset of active gradients; aliasing,
determinism and autocast float32 bias; the error contract.  Tolerances are
those of the triangle tests (fp32 1e-5, 16-bit 2e-2 scaled max-abs and 1e-2
mean-relative against the float64 oracle on the same rounded inputs).
"""

import numpy as np
import pytest
import torch

from oracle import attention as ora
from oops_amd import OOpsUnsupportedError, pair_bias_attention

from accuracy import assert_close

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _np(t):
    return None if t is None else t.detach().double().cpu().numpy()


def make_inputs(dtype, *, layout="dense", lengths=(33, 35), head_size=24, heads=2, mask_kind="pair",
                bias_kind="full", seed=0):
    """Reference-shaped inputs (test_pair_bias_attention.py:23-35, :246-268) on the GPU."""

    g = torch.Generator().manual_seed(seed)
    prefix = (2, 3) if layout == "sampled" else (2,)
    rows, cols = lengths
    q = torch.randn((*prefix, heads, rows, head_size), generator=g).to(dtype)
    k, v = (torch.randn((*prefix, heads, cols, head_size), generator=g).to(dtype) for _ in range(2))
    q, k, v = (t.to(DEV) for t in (q, k, v))
    if layout == "sliced":
        q, k, v = (torch.stack((t, t), -1)[..., 0] for t in (q, k, v))
    shape = (*prefix, cols) if mask_kind == "key" else (*prefix, rows, cols)
    mask = None
    if mask_kind != "none":
        mask = torch.rand(shape, generator=g) > 0.2
        mask[..., 0] = True
        mask = mask.to(DEV)
    bias = None
    if bias_kind != "none":
        bias_prefix = (*prefix[:-1], 1) if bias_kind == "shared" and len(prefix) > 1 else prefix
        if bias_kind == "shared" and len(prefix) == 1:
            bias_prefix = (1,)
        bias = torch.randn((*bias_prefix, heads, rows, cols), generator=g).to(dtype).to(DEV)
    return q, k, v, mask, bias


def check(q, k, v, mask, bias, dtype, *, scale=None, active=("query", "key", "value", "bias"), negative=False,
          tol16=2e-2):
    leaves_by_name = {}
    tensors = []
    for name, t in zip(("query", "key", "value", "bias"), (q, k, v, bias)):
        if t is None:
            tensors.append(None)
            continue
        t = t.detach().clone().requires_grad_(name in active)
        if name in active:
            leaves_by_name[name] = t
        tensors.append(t)
    call = [torch._neg_view(t) if (negative and t is not None) else t for t in tensors]
    out = pair_bias_attention(call[0], call[1], call[2], mask, call[3], scale=scale)
    assert out.shape == q.shape and out.dtype == q.dtype
    sign = -1.0 if negative else 1.0
    nq, nk, nv, nb = (None if t is None else sign * _np(t) for t in tensors)
    assert_close(out, ora.pair_bias_attention_forward(nq, nk, nv, _np(mask), nb, scale), dtype, "out", tol16)
    if not leaves_by_name:
        return
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(7)).to(dtype).to(DEV)
    names = list(leaves_by_name)
    got = torch.autograd.grad(out, [leaves_by_name[n] for n in names], dout)
    want = dict(zip(("query", "key", "value", "bias"),
                    ora.pair_bias_attention_backward(nq, nk, nv, _np(dout), _np(mask), nb, scale)))  # fmt: skip
    for name, g_ in zip(names, got):
        leaf = leaves_by_name[name]
        assert g_.shape == leaf.shape and g_.dtype == leaf.dtype, name
        assert_close(g_, sign * want[name], dtype, "d" + name, tol16)


@pytest.mark.parametrize(
    "dtype,layout,mask_kind,bias_kind,lengths,scale",
    [
        (torch.float32, "dense", "pair", "none", (33, 35), 0.25),
        (torch.float32, "dense", "none", "none", (1, 31), 0.25),
        (torch.float32, "negative", "pair", "full", (33, 35), 0.25),
        (torch.float16, "sliced", "key", "full", (33, 35), 0.25),
        (torch.bfloat16, "sampled", "pair", "shared", (31, 129), 0.25),
        (torch.bfloat16, "dense", "key", "full", (64, 200), None),
        (torch.bfloat16, "sampled", "key", "shared", (130, 64), None),
        (torch.float16, "dense", "none", "shared", (96, 96), None),
    ],
)
def test_forward_backward(dtype, layout, mask_kind, bias_kind, lengths, scale):
    q, k, v, mask, bias = make_inputs(dtype, layout=layout, lengths=lengths, mask_kind=mask_kind,
                                      bias_kind=bias_kind)  # fmt: skip
    check(q, k, v, mask, bias, dtype, scale=scale, negative=layout == "negative")


@pytest.mark.parametrize(
    "dtype,mask_kind,bias_kind,active,shape",
    [
        (torch.float32, "pair", "full", ("query", "key", "value", "bias"), (33, 129, 24)),
        (torch.float32, "pair", "none", ("query", "key", "value"), (17, 19, 16)),
        (torch.bfloat16, "pair", "full", ("query", "value"), (33, 129, 24)),
        (torch.float32, "pair", "shared", ("bias",), (33, 129, 24)),
        (torch.bfloat16, "none", "none", ("key",), (33, 129, 24)),
        (torch.float32, "pair", "shared", ("query", "key", "value", "bias"), (128, 128, 128)),
        (torch.bfloat16, "key", "full", ("query", "key", "value", "bias"), (128, 256, 32)),
        (torch.bfloat16, "key", "shared", ("query", "key", "value", "bias"), (384, 384, 64)),
    ],
)
def test_backward_subsets(dtype, mask_kind, bias_kind, active, shape):
    q, k, v, mask, bias = make_inputs(dtype, lengths=shape[:2], head_size=shape[2], mask_kind=mask_kind,
                                      bias_kind=bias_kind, seed=shape[0])  # fmt: skip
    check(q, k, v, mask, bias, dtype, scale=0.25, active=active)


@pytest.mark.parametrize("bias_shape", [(1, 2, 1, 35), (2, 1, 33, 35), (2, 2, 33, 1), (1, 1, 1, 1)])
def test_broadcast_bias(bias_shape):
    """Bias broadcast over heads/queries/keys; its gradient is summed to its own shape."""

    q, k, v, mask, _ = make_inputs(torch.float32, mask_kind="key", bias_kind="none", seed=11)
    bias = torch.randn(bias_shape, generator=torch.Generator().manual_seed(3)).to(DEV)
    check(q, k, v, mask, bias, torch.float32)


def test_rank3_and_mask_head_axis():
    q, k, v, mask, bias = make_inputs(torch.float32, lengths=(9, 12), seed=5)
    q3, k3, v3, b3 = q[0], k[0], v[0], bias[0]
    m3 = mask[0]
    check(q3, k3, v3, m3, b3, torch.float32)
    # a unit head axis before the query axis, and a unit query axis (key mask in pair form)
    check(q, k, v, mask[:, None], bias, torch.float32)
    check(q, k, v, mask[:, :1], bias, torch.float32)


def test_prefixed_rank6():
    g = torch.Generator().manual_seed(9)
    q, k, v = (torch.randn(2, 2, 3, 2, 10, 16, generator=g).to(DEV) for _ in range(3))
    mask = (torch.rand(2, 2, 3, 10, generator=g) > 0.3).to(DEV)
    bias = torch.randn(2, 2, 1, 2, 10, 10, generator=g).to(DEV)
    check(q, k, v, mask, bias, torch.float32)


def test_fully_masked_rows():
    q, k, v, mask, bias = make_inputs(torch.float32, seed=2)
    mask[0, 3] = False
    check(q, k, v, mask, bias, torch.float32)
    mask.zero_()
    out = pair_bias_attention(q, k, v, mask, bias)
    torch.testing.assert_close(out, torch.zeros_like(out))


def test_alias_and_determinism():
    q, _, _, mask, bias = make_inputs(torch.float32, lengths=(33, 33), seed=4)
    qd = q.clone().requires_grad_(True)
    bd = bias.clone().requires_grad_(True)
    out = pair_bias_attention(qd, qd, qd, mask, bd)
    dout = torch.randn_like(out)
    g1 = torch.autograd.grad(out, (qd, bd), dout, retain_graph=True)
    g2 = torch.autograd.grad(out, (qd, bd), dout)
    for a, b in zip(g1, g2):
        torch.testing.assert_close(a, b, atol=0, rtol=0)
    nq, nb = _np(q), _np(bias)
    dq, dk, dv, db = ora.pair_bias_attention_backward(nq, nq, nq, _np(dout), _np(mask), nb)
    assert_close(g1[0], dq + dk + dv, torch.float32, "alias dq")
    assert_close(g1[1], db, torch.float32, "alias dbias")


def test_autocast_float32_bias():
    q, k, v, mask, bias = make_inputs(torch.bfloat16, seed=6)
    bias32 = bias.float().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = pair_bias_attention(q, k, v, mask, bias32)
    assert out.dtype == torch.bfloat16
    want = ora.pair_bias_attention_forward(_np(q), _np(k), _np(v), _np(mask), _np(bias32))
    assert_close(out, want, torch.bfloat16, "out")
    (gb,) = torch.autograd.grad(out, (bias32,), torch.ones_like(out))
    assert gb.dtype == torch.float32
    # outside autocast a float32 bias over bf16 q/k/v is refused (reference problem.py:240-251)
    with pytest.raises(OOpsUnsupportedError):
        pair_bias_attention(q, k, v, mask, bias32)


def test_config_c4_msa_rows():
    """BASELINE config 4 at full size: S=512, H=8, N=384, c=32 bf16, key mask, shared bias (seed 3).

    Groups are independent, so the oracle checks O, dQ, dK and dV on a slice of 16 sequences of the
    full-size call; the shared dBias (a sum over all 512 groups) on a query subset over every group.
    """

    torch.manual_seed(3)
    s, h, n, c = 512, 8, 384, 32
    q, k, v = (torch.randn(s, n, h, c).to(torch.bfloat16).permute(0, 2, 1, 3).to(DEV) for _ in range(3))
    bias = torch.randn(1, h, n, n).to(torch.bfloat16).to(DEV)
    mask = torch.rand(s, n) > 0.15
    mask[:, 0] = True
    mask = mask.to(DEV)
    dout = torch.randn(s, h, n, c).to(torch.bfloat16).to(DEV)
    leaves = [t.requires_grad_(True) for t in (q, k, v, bias)]
    out = pair_bias_attention(q, k, v, mask, bias)
    gq, gk, gv, gb = torch.autograd.grad(out, leaves, dout)
    sl = slice(100, 116)
    nb = _np(bias)
    want_o = ora.pair_bias_attention_forward(_np(q[sl]), _np(k[sl]), _np(v[sl]), _np(mask[sl]), nb)
    assert_close(out[sl], want_o, torch.bfloat16, "out")
    dq, dk, dv, _ = ora.pair_bias_attention_backward(_np(q[sl]), _np(k[sl]), _np(v[sl]), _np(dout[sl]),
                                                     _np(mask[sl]), nb)  # fmt: skip
    assert_close(gq[sl], dq, torch.bfloat16, "dq")
    assert_close(gk[sl], dk, torch.bfloat16, "dk")
    assert_close(gv[sl], dv, torch.bfloat16, "dv")
    # dBias sums over all 512 groups: the float64 oracle over every group, on 48 query positions spread
    # over all twelve 32-query tiles (exact for those queries: each is its own softmax)
    qpos = [32 * t + (7 * j + t) % 32 for t in range(12) for j in range(4)]
    f32 = lambda t: t.detach().float().cpu().numpy()  # noqa: E731
    want_db = ora.shared_dbias_at(f32(q), f32(k), f32(v), f32(dout), _np(mask), nb, qpos)
    assert_close(gb[0][:, qpos], want_db, torch.bfloat16, "dbias")


def test_errors():
    q = torch.randn(2, 2, 5, 8, device=DEV)
    with pytest.raises(ValueError):
        pair_bias_attention(q, q, q[..., :-1])
    with pytest.raises(OOpsUnsupportedError):
        pair_bias_attention(q.double(), q.double(), q.double())
    with pytest.raises(OOpsUnsupportedError):  # mask head axis of size 2
        pair_bias_attention(q, q, q, torch.ones(2, 2, 5, 5, dtype=torch.bool, device=DEV))
    with pytest.raises(OOpsUnsupportedError):  # non-bool mask
        pair_bias_attention(q, q, q, torch.ones(2, 5, device=DEV))
    with pytest.raises(OOpsUnsupportedError):  # bias batch mismatch
        pair_bias_attention(q, q, q, None, torch.randn(3, 2, 5, 5, device=DEV))


@pytest.mark.parametrize("dout_layout", ["contiguous", "output"])
def test_dout_layout_independent(dout_layout):
    """dO in its own layout (read through remapped table columns) gives the same gradients, bit for bit."""

    g = torch.Generator().manual_seed(11)
    s_, n, h, c = 6, 70, 4, 32
    q, k, v = (torch.randn(s_, n, h, c, generator=g).to(torch.bfloat16).permute(0, 2, 1, 3).to(DEV)
               for _ in range(3))  # fmt: skip
    mask = (torch.rand(s_, n, generator=g) > 0.2).to(DEV)
    bias = torch.randn(1, h, n, n, generator=g).to(torch.bfloat16).to(DEV)
    base = torch.randn(s_, h, n, c, generator=g).to(torch.bfloat16)
    dout = base.to(DEV) if dout_layout == "contiguous" else base.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3).to(DEV)
    results = []
    for d in (dout, torch.empty_strided(q.shape, q.stride(), dtype=q.dtype, device=DEV).copy_(dout)):
        leaves = [t.detach().clone().requires_grad_(True) for t in (q, k, v, bias)]
        out = pair_bias_attention(leaves[0], leaves[1], leaves[2], mask, leaves[3])
        results.append(torch.autograd.grad(out, leaves, d))
    for got, want in zip(*results):
        torch.testing.assert_close(got, want, rtol=0, atol=0)
