"""Gated output stage on the GPU against the float64 oracle (oracle/gate.py).

Mirrors the reference's gate tests (tests/attention/gate/*): dense ranks 3-5,
the fused 16-bit projection kernel (head size a multiple of 16) and the
unfused path (logits by F.linear, the HIP elementwise kernel), fp32, nested
values with the token-major packing, gated_pair_bias_attention end to end,
and torch.compile.
"""

import numpy as np
import pytest
import torch

from accuracy import assert_close
from oracle import attention as ora
from oracle import gate as gora
from oops_amd import gate_attention_output, gated_pair_bias_attention

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _np(t):
    return t.detach().double().cpu().numpy()


_ROUNDING = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: None}


def _inputs(dtype, prefix, heads, q, d, c, o, seed):
    g = torch.Generator().manual_seed(seed)
    att = torch.randn(*prefix, heads, q, d, generator=g).to(dtype)
    single = torch.randn(*prefix, q, c, generator=g).to(dtype)
    w = (torch.randn(heads * d, c, generator=g) / c**0.5).to(dtype)
    wo = (torch.randn(o, heads * d, generator=g) / (heads * d) ** 0.5).to(dtype)
    dy = torch.randn(*prefix, q, o, generator=g).to(dtype)
    return att, single, w, wo, dy


def _check(att, single, w, wo, dy, dtype):
    leaves = [t.to(DEV).requires_grad_(True) for t in (att, single, w, wo)]
    out = gate_attention_output(*leaves)
    rnd = _ROUNDING[dtype]
    want_out, _, _ = gora.gate_attention_output_forward(*(_np(t) for t in (att, single, w, wo)), rounding=rnd)
    assert out.dtype == dtype and out.shape == tuple(want_out.shape)
    assert_close(out, want_out, dtype, "out")
    grads = torch.autograd.grad(out, leaves, dy.to(DEV))
    want = gora.gate_attention_output_backward(*(_np(t) for t in (att, single, w, wo, dy)), rounding=rnd)
    for name, got, ref in zip(("attention", "single", "gate_weight", "output_weight"), grads, want):
        assert got.shape == tuple(ref.shape), name
        assert_close(got, ref, dtype, name)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("prefix", [(), (3,), (2, 3)])
@pytest.mark.parametrize("d", [32, 24])  # 32: fused projection kernel (16-bit); 24: F.linear + elementwise kernel
def test_gate_dense(dtype, prefix, d):
    _check(*_inputs(dtype, prefix, heads=4, q=37, d=d, c=72, o=40, seed=len(prefix) + d), dtype)


@pytest.mark.parametrize(
    "dtype,prefix,heads,q,c",
    [
        (torch.bfloat16, (171,), 4, 397, 160),  # three k panels (run as four), two token tiles per workgroup, ragged end
        (torch.float16, (5,), 2, 33, 64),  # one k panel, a partial channel tile (N = 64)
        (torch.bfloat16, (3,), 12, 50, 320),  # C > 256: the streaming projection kernel
    ],
)
def test_gate_projection_forms(dtype, prefix, heads, q, c):
    """The W-resident projection (C <= 256, workgroups walking runs of token tiles) and the streaming one."""

    _check(*_inputs(dtype, prefix, heads=heads, q=q, d=32, c=c, o=48, seed=c + q), dtype)


def test_gate_large_msa_shape():
    """MSA-row shape (S=64, N=384, H=8, c=32, C=256, O=256), bf16."""

    _check(*_inputs(torch.bfloat16, (64,), heads=8, q=384, d=32, c=256, o=256, seed=7), torch.bfloat16)


def test_gate_strided_attention():
    """Attention read through its strides: a (Q, H, D)-major buffer viewed head-major."""

    att, single, w, wo, dy = _inputs(torch.bfloat16, (3,), heads=4, q=40, d=32, c=64, o=16, seed=3)
    att_strided = att.transpose(-3, -2).contiguous().transpose(-3, -2)  # same values, token-major memory
    assert not att_strided.is_contiguous()
    _check(att_strided, single, w, wo, dy, torch.bfloat16)


class _Packed:
    """Minimal token-major NestedTensor stand-in for the gate (DanLing's packing)."""

    def __init__(self, concat, lengths, ragged_dims, packed_dim_order, ndim):
        self.concat = concat
        self._lengths = lengths
        self.ragged_dims = ragged_dims
        self.packed_dim_order = packed_dim_order
        self.batch_first = True
        self._ndim = ndim

    def dim(self):
        return self._ndim

    def packed_like(self, values):
        return _Packed(values, self._lengths, self.ragged_dims, self.packed_dim_order, self._ndim)

    def packed_offsets(self, dtype=torch.int64, device=None):
        return torch.tensor([0, *np.cumsum(self._lengths)], dtype=dtype, device=device)

    def packed_with_static_tail(self, values):
        return self.packed_like(values)


@pytest.mark.parametrize("explicit_s", [False, True])
def test_gate_nested(explicit_s):
    g = torch.Generator().manual_seed(5)
    lengths = (13, 40, 7)
    s_, h, d, c, o = (2 if explicit_s else 1), 4, 32, 48, 24
    n = sum(lengths)
    att = torch.randn(n, s_, h, d, generator=g).to(torch.bfloat16)
    single = torch.randn(n, s_, c, generator=g).to(torch.bfloat16)
    w = (torch.randn(h * d, c, generator=g) / c**0.5).to(torch.bfloat16)
    wo = (torch.randn(o, h * d, generator=g) / (h * d) ** 0.5).to(torch.bfloat16)
    if explicit_s:
        na = _Packed(att.to(DEV), lengths, (2,), (2, 0, 1, 3), 5)
        ns = _Packed(single.to(DEV), lengths, (1,), (1, 0, 2), 4)
    else:
        na = _Packed(att[:, 0].to(DEV), lengths, (1,), (1, 0, 2), 4)
        ns = _Packed(single[:, 0].to(DEV), lengths, (0,), (0, 1), 3)
    out = gate_attention_output(na, ns, w.to(DEV), wo.to(DEV))
    # packed rows (token t, group s): attention (H, D), single (C); the oracle
    # takes them as prefix = S, Q = tokens
    want, _, _ = gora.gate_attention_output_forward(
        np.transpose(_np(att), (1, 2, 0, 3)), np.transpose(_np(single), (1, 0, 2)), _np(w), _np(wo), rounding="bf16")
    want = np.transpose(want, (1, 0, 2))  # (tokens, S, O)
    got = out.concat if explicit_s else out.concat[:, None]
    assert_close(got, want, torch.bfloat16, "nested out")


def test_gated_pair_bias_attention():
    g = torch.Generator().manual_seed(9)
    s_, h, n, d, c, o = 4, 4, 50, 32, 64, 32
    q, k, v = (torch.randn(s_, h, n, d, generator=g).to(torch.bfloat16) for _ in range(3))
    mask = torch.rand(s_, n, generator=g) > 0.2
    bias = torch.randn(1, h, n, n, generator=g).to(torch.bfloat16)
    single = torch.randn(s_, n, c, generator=g).to(torch.bfloat16)
    w = (torch.randn(h * d, c, generator=g) / c**0.5).to(torch.bfloat16)
    wo = (torch.randn(o, h * d, generator=g) / (h * d) ** 0.5).to(torch.bfloat16)
    out = gated_pair_bias_attention(single.to(DEV), q.to(DEV), k.to(DEV), v.to(DEV), mask.to(DEV),
                                    pair_bias=bias.to(DEV), gate_weight=w.to(DEV), output_weight=wo.to(DEV))
    att = ora.pair_bias_attention_forward(_np(q), _np(k), _np(v), _np(mask), _np(bias), d**-0.5)
    # the attention output is stored in bf16 before the gate
    att = gora._rounder("bf16")(att)
    want, _, _ = gora.gate_attention_output_forward(att, _np(single), _np(w), _np(wo), rounding="bf16")
    assert_close(out, want, torch.bfloat16, "gated pair-bias out")
    with pytest.raises(ValueError):
        gated_pair_bias_attention(single.to(DEV), q.to(DEV), k.to(DEV), v.to(DEV), gate_weight=w.to(DEV),
                                  output_weight=wo.to(DEV))


def test_gate_compile_matches_eager():
    att, single, w, wo, dy = _inputs(torch.bfloat16, (2,), heads=4, q=33, d=32, c=64, o=16, seed=11)

    def run(a, s, w_, wo_):
        return gate_attention_output(a, s, w_, wo_)

    results = []
    for fn in (run, torch.compile(run, fullgraph=True)):
        leaves = [t.to(DEV).requires_grad_(True) for t in (att, single, w, wo)]
        out = fn(*leaves)
        results.append((out.detach(), *torch.autograd.grad(out, leaves, dy.to(DEV))))
    for got, ref in zip(*results):
        torch.testing.assert_close(got, ref, atol=0, rtol=0)


def test_gate_errors():
    att, single, w, wo, _ = _inputs(torch.bfloat16, (2,), heads=4, q=8, d=32, c=16, o=8, seed=1)
    att, single, w, wo = (t.to(DEV) for t in (att, single, w, wo))
    with pytest.raises(ValueError):
        gate_attention_output(att, single[..., :-1], w, wo)
    with pytest.raises(ValueError):
        gate_attention_output(att, single, w[:-1], wo)
    with pytest.raises(ValueError):
        gate_attention_output(att[0, 0], single, w, wo)
