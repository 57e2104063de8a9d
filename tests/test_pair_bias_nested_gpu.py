"""GPU parity of nested (ragged MSA) pair-bias attention against the numpy oracle.

Follows the reference's nested pair-bias cases
(tests/attention/pair_bias/test_pair_bias_attention.py:57-226, :330-487):
implicit, static, doubly ragged group-outer / token-outer ("column") and
ragged-group packings; key, per-group key and pair masks; shared, per-group
and head-shared bias; rectangular Q/K; gradients of the packed q/k/v and bias
values.  Expected values: the dense oracle per sample, packed back with the
operand's own topology.
"""

import pytest
import torch

from accuracy import assert_close
from nested_pair_cases import expected_grads, expected_outputs, make_case
from nested_standin import NestedTensor
from oops_amd import OOpsUnsupportedError, gated_pair_bias_attention, pair_bias_attention
from oracle import attention as ora
from oracle import gate as gora

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _np(t):
    return t.detach().double().cpu().numpy()


CASES = [
    # layout, mask kind, mask shared, bias kind
    ("implicit", "key", True, "full"),
    ("implicit", "pair", True, "shared_head"),
    ("static", "pair", True, "shared"),
    ("static", "key", False, "full"),
    ("static", "key_singleton", False, "shared_head"),
    ("group_outer", "key", False, "shared"),
    ("group_outer", "pair", True, "shared_head"),
    ("token_outer", "key", False, "none"),
    ("token_outer", "key", True, "shared"),
    ("ragged_groups", "key", False, "shared_head"),
    ("ragged_groups", "none", True, "none"),
    ("ragged_groups_tokens", "key", False, "shared"),
]


def _check(case_inputs, leaves, dtype, scale=None):
    q, k, v, mask, bias = case_inputs
    out = pair_bias_attention(q, k, v, mask, bias, scale=scale)
    assert isinstance(out, NestedTensor)
    assert out.concat.shape == q.concat.shape and out.concat.dtype == dtype
    want = expected_outputs(q, k, v, mask, bias, scale)
    for i, (g_, w_) in enumerate(zip(out.unbind(), want)):
        assert_close(g_, w_, dtype, f"out[{i}]")
    douts = [torch.randn(o.shape, generator=torch.Generator().manual_seed(3 + i)).to(dtype).to(DEV)
             for i, o in enumerate(out.unbind())]  # fmt: skip
    dout = torch.cat([q._pack(d) for d in douts])
    leaves = [t for t in leaves if t is not None]
    got = torch.autograd.grad(out.concat, leaves, dout)
    want_g = [t for t in expected_grads(q, k, v, mask, bias, douts, scale) if t is not None]
    for name, g_, w_ in zip(("dq", "dk", "dv", "dbias"), got, want_g):
        assert g_.shape == w_.shape, name
        assert_close(g_, w_.numpy(), dtype, name)


@pytest.mark.parametrize("layout,mask_kind,mask_shared,bias_kind", CASES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_nested_pair_bias(layout, mask_kind, mask_shared, bias_kind, dtype):
    small = dtype == torch.float32
    inputs, leaves = make_case(
        layout, dtype=dtype, device=DEV, mask_kind=mask_kind, mask_shared=mask_shared, bias_kind=bias_kind,
        q_lengths=(5, 9) if small else (33, 70), k_lengths=(7, 4) if small else (41, 64),
        groups=(2, 3) if layout != "static" else (3, 3), heads=2 if small else 4, head_size=16 if small else 32,
        seed=len(layout) + len(mask_kind), requires_grad=True,
    )  # fmt: skip
    _check(inputs, leaves, dtype, scale=None if small else 0.25)


@pytest.mark.parametrize("head_size", [24, 64])
def test_nested_pair_bias_head_sizes(head_size):
    inputs, leaves = make_case("group_outer", dtype=torch.float16, device=DEV, q_lengths=(40, 17),
                               k_lengths=(40, 17), groups=(3, 2), heads=2, head_size=head_size, mask_kind="key",
                               mask_shared=False, bias_kind="shared", seed=head_size, requires_grad=True)  # fmt: skip
    _check(inputs, leaves, torch.float16)


def test_nested_matches_dense():
    """A one-sample static nested call equals the dense call on the same element."""

    (q, k, v, mask, bias), _ = make_case("static", dtype=torch.bfloat16, device=DEV, q_lengths=(48,),
                                         k_lengths=(48,), groups=(3,), heads=4, head_size=32, mask_kind="key",
                                         bias_kind="shared", seed=8)  # fmt: skip
    out = pair_bias_attention(q, k, v, mask, bias)
    qd, kd, vd, md, bd = (torch.unbind(t)[0] for t in (q, k, v, mask, bias))
    dense = pair_bias_attention(qd, kd, vd, md, bd)
    torch.testing.assert_close(out.unbind()[0], dense, atol=0, rtol=0)


def test_nested_msa_scale():
    """MSA-sized ragged batch: S_i in {64, 128} sequences, N_i in {256, 384}, H=8, c=32, bf16, shared
    bias and per-group key masks, doubly ragged (group-outer) packing.  The oracle checks 2 sequences
    of every sample (sequences are independent); the shared dBias sums every sequence and is checked
    against a float32 torch restatement over all of them."""

    dtype = torch.bfloat16
    inputs, leaves = make_case("group_outer", dtype=dtype, device=DEV, q_lengths=(256, 384), k_lengths=(256, 384),
                               groups=(64, 128), heads=8, head_size=32, mask_kind="key", mask_shared=False,
                               bias_kind="shared", seed=2, requires_grad=True)  # fmt: skip
    q, k, v, mask, bias = inputs
    out = pair_bias_attention(q, k, v, mask, bias)
    dout_parts = [torch.randn(o.shape, generator=torch.Generator().manual_seed(7)).to(dtype).to(DEV)
                  for o in out.unbind()]  # fmt: skip
    grads = torch.autograd.grad(out.concat, list(leaves), torch.cat([q._pack(d) for d in dout_parts]))
    dbias_parts = bias.packed_like(grads[3]).unbind()
    for i, (qe, ke, ve, me, be, oe, de) in enumerate(
        zip(q.unbind(), k.unbind(), v.unbind(), mask.unbind(), bias.unbind(), out.unbind(), dout_parts)
    ):
        rows = [0, qe.shape[0] - 1]
        ref = ora.pair_bias_attention_forward(*(_np(t[rows]) for t in (qe, ke, ve, me)), _np(be))
        assert_close(oe[rows], ref, dtype, f"out[{i}]")
        # shared dBias over every sequence, float32 torch restatement
        qf, kf, vf, bf, df = (t.detach().float() for t in (qe, ke, ve, be, de))
        s = qf @ kf.transpose(-1, -2) * qe.shape[-1] ** -0.5 + bf
        keep = me[:, :, None, :]
        s = s.masked_fill(~keep, float("-inf"))
        p = torch.softmax(s, -1).nan_to_num(0.0)
        o = p @ vf
        dp = df @ vf.transpose(-1, -2)
        ds = p * (dp - (df * o).sum(-1, keepdim=True))
        assert_close(dbias_parts[i], ds.sum(0, keepdim=True).double().cpu().numpy(), dtype, f"dbias[{i}]")


def test_gated_nested_pair_bias():
    """gated_pair_bias_attention over a static-group nested batch: attention then the gate."""

    dtype = torch.bfloat16
    (q, k, v, mask, bias), _ = make_case("static", dtype=dtype, device=DEV, q_lengths=(20, 33), k_lengths=(20, 33),
                                         groups=(2, 2), heads=4, head_size=32, mask_kind="key", bias_kind="shared",
                                         seed=12)  # fmt: skip
    g = torch.Generator().manual_seed(1)
    c, o = 48, 24
    single_tmpl = NestedTensor([torch.empty(2, n, c) for n in (20, 33)], ragged_dims=(1,))
    single = single_tmpl.packed_like(torch.randn(single_tmpl.concat.shape, generator=g).to(dtype).to(DEV))
    w = (torch.randn(4 * 32, c, generator=g) / c**0.5).to(dtype).to(DEV)
    wo = (torch.randn(o, 4 * 32, generator=g) / 128**0.5).to(dtype).to(DEV)
    out = gated_pair_bias_attention(single, q, k, v, mask, bias, gate_weight=w, output_weight=wo)
    att = pair_bias_attention(q, k, v, mask, bias)
    for i, (ae, se, oe) in enumerate(zip(att.unbind(), single.unbind(), out.unbind())):
        want, _, _ = gora.gate_attention_output_forward(_np(ae), _np(se), _np(w), _np(wo), rounding="bf16")
        assert_close(oe, want, dtype, f"gated[{i}]")


def test_nested_errors_gpu():
    (q, k, v, mask, bias), _ = make_case("static", dtype=torch.float32, device=DEV)
    with pytest.raises(OOpsUnsupportedError):
        pair_bias_attention(*(t.packed_like(t.concat.double()) for t in (q, k, v)))
    with pytest.raises(ValueError):
        pair_bias_attention(q, k, v.packed_like(v.concat[:, :1].contiguous()))
