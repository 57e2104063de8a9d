"""Seeded random-shape parity sweeps of the rows beside attention.

Each case draws its sizes, layout, mask and bias options from a fixed seed
and checks the HIP path against the float64 oracle, so odd combinations that
the hand-picked tests do not name (widths not multiples of 8 or 16, a single
token, prefixes, ragged packings) are exercised on every run.
"""

import numpy as np
import pytest
import torch

from accuracy import assert_close
from nested_pair_cases import LAYOUTS, expected_grads, expected_outputs, make_case
from oops_amd import gate_attention_output, pair_bias_attention, triangle_multiplication
from oracle import gate as gora
from oracle import trimul as otm

pytestmark = pytest.mark.gpu

DEV = "cuda"
_ROUND = {torch.bfloat16: "bf16", torch.float16: "f16"}
_NAMES = ("input_norm_weight", "input_norm_bias", "left_value_weight", "left_gate_weight", "right_value_weight",
          "right_gate_weight", "output_norm_weight", "output_norm_bias", "output_weight", "output_gate_weight")
_BIAS = ("left_value_bias", "left_gate_bias", "right_value_bias", "right_gate_bias", "output_bias",
         "output_gate_bias")  # fmt: skip


def _np(t):
    return None if t is None else t.detach().double().cpu().numpy()


def _grad_close(got, want, tol, what):
    err = np.abs(_np(got) - want).max()
    assert err <= tol * max(1.0, float(np.abs(want).max())), f"{what}: {err:.3g}"


@pytest.mark.parametrize("seed", range(10))
def test_trimul_random(seed):
    rng = np.random.default_rng(100 + seed)
    dtype = [torch.bfloat16, torch.float16][seed % 2]
    # 16-bit widths of at least 8, as in the reference's 16-bit cases: with one or two channels a
    # LayerNorm's gradient cancels to near zero and multiplies the operands' 2^-9 rounding by its 1/std
    c, h, n = int(rng.integers(8, 70)), int(rng.integers(8, 70)), int(rng.integers(1, 24))
    prefix = tuple(int(x) for x in rng.integers(1, 3, size=int(rng.integers(0, 3))))
    direction = ["outgoing", "incoming"][int(rng.integers(0, 2))]
    g = torch.Generator().manual_seed(seed)

    def r(*shape, scale=1.0, dt=dtype):
        return (torch.randn(*shape, generator=g) * scale).to(dt).to(DEV).requires_grad_(True)

    pair = r(*prefix, n, n, c)
    mask = (torch.rand(*prefix, n, n, generator=g) > 0.3).to(DEV) if seed % 3 else None
    weights = (r(c), r(c), r(h, c, scale=c**-0.5), r(h, c, scale=c**-0.5), r(h, c, scale=c**-0.5),
               r(h, c, scale=c**-0.5), r(h), r(h), r(c, h, scale=h**-0.5), r(c, c, scale=c**-0.5))  # fmt: skip
    bs = tuple(r(w, scale=0.2) for w in (h, h, h, h, c, c)) if seed % 2 else (None,) * 6
    kw = dict(zip(_NAMES, weights))
    kw.update(dict(zip(_BIAS, bs)))
    out = triangle_multiplication(pair, mask, direction=direction, **kw)
    np_w, np_b = [_np(w) for w in weights], [_np(b) for b in bs]
    want = otm.triangle_multiplication_forward(_np(pair), _np(mask), np_w, np_b, direction, rounding=_ROUND[dtype])
    assert_close(out, want, dtype, f"out (C={c}, H={h}, N={n}, prefix={prefix})")
    dy = torch.randn(out.shape, generator=g).to(dtype).to(DEV)
    got = torch.autograd.grad(out, [pair, weights[2], weights[8]], dy)
    d_pair, _, d_w, _ = otm.triangle_multiplication_backward(_np(pair), _np(mask), np_w, np_b, _np(dy), direction)
    tol = 5e-2 if dtype == torch.bfloat16 else 3e-2
    for name, got_, want_ in zip(("pair", "left_value_weight", "output_weight"), got, (d_pair, d_w[2], d_w[8])):
        _grad_close(got_, want_, tol, name)


@pytest.mark.parametrize("seed", range(10))
def test_nested_pair_bias_random(seed):
    rng = np.random.default_rng(200 + seed)
    layout = LAYOUTS[seed % len(LAYOUTS)]
    dtype = torch.bfloat16
    n_samples = int(rng.integers(1, 4))
    q_lengths = tuple(int(x) for x in rng.integers(1, 40, size=n_samples))
    k_lengths = tuple(int(x) for x in rng.integers(1, 40, size=n_samples))
    groups = tuple(int(x) for x in rng.integers(1, 4, size=n_samples))
    grouped = layout not in ("implicit", "static")
    mask_kind = ["none", "key", "pair"][int(rng.integers(0, 3))]
    if grouped and layout.startswith("ragged") and mask_kind == "pair":
        mask_kind = "key"
    mask_shared = bool(rng.integers(0, 2)) if not grouped else (mask_kind != "key" or bool(rng.integers(0, 2)))
    if grouped and mask_kind == "pair":
        mask_shared = True
    bias_kind = ["none", "shared", "shared_head"][int(rng.integers(0, 3))]
    head_size = [8, 16, 24, 32][int(rng.integers(0, 4))]
    inputs, leaves = make_case(layout, dtype=dtype, device=DEV, q_lengths=q_lengths, k_lengths=k_lengths,
                               groups=groups if layout != "static" else (groups[0],) * n_samples,
                               heads=int(rng.integers(1, 4)), head_size=head_size, mask_kind=mask_kind,
                               mask_shared=mask_shared, bias_kind=bias_kind, seed=seed, requires_grad=True)  # fmt: skip
    q, k, v, mask, bias = inputs
    out = pair_bias_attention(q, k, v, mask, bias)
    for i, (g_, w_) in enumerate(zip(out.unbind(), expected_outputs(q, k, v, mask, bias))):
        assert_close(g_, w_, dtype, f"{layout} out[{i}]")
    douts = [torch.randn(o.shape, generator=torch.Generator().manual_seed(seed + i)).to(dtype).to(DEV)
             for i, o in enumerate(out.unbind())]  # fmt: skip
    leaves = [t for t in leaves if t is not None]
    got = torch.autograd.grad(out.concat, leaves, torch.cat([q._pack(d) for d in douts]))
    want = [t for t in expected_grads(q, k, v, mask, bias, douts) if t is not None]
    for name, g_, w_ in zip(("dq", "dk", "dv", "dbias"), got, want):
        assert_close(g_, w_.numpy(), dtype, f"{layout} {name}")


@pytest.mark.parametrize("seed", range(6))
def test_gate_random(seed):
    rng = np.random.default_rng(300 + seed)
    dtype = [torch.bfloat16, torch.float16][seed % 2]
    heads, width = int(rng.integers(1, 5)), [8, 16, 24, 32, 48][int(rng.integers(0, 5))]
    c, o, q = int(rng.integers(1, 80)), int(rng.integers(1, 40)), int(rng.integers(1, 50))
    prefix = tuple(int(x) for x in rng.integers(1, 3, size=int(rng.integers(0, 3))))
    g = torch.Generator().manual_seed(seed)
    att = torch.randn(*prefix, heads, q, width, generator=g).to(dtype).to(DEV)
    single = torch.randn(*prefix, q, c, generator=g).to(dtype).to(DEV)
    w = (torch.randn(heads * width, c, generator=g) / c**0.5).to(dtype).to(DEV)
    wo = (torch.randn(o, heads * width, generator=g) / (heads * width) ** 0.5).to(dtype).to(DEV)
    out = gate_attention_output(att, single, w, wo)
    want, _, _ = gora.gate_attention_output_forward(_np(att), _np(single), _np(w), _np(wo), rounding=_ROUND[dtype])
    assert_close(out, want, dtype, f"gate (H={heads}, D={width}, C={c}, O={o}, Q={q}, prefix={prefix})")
