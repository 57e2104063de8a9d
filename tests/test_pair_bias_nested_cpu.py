"""Host logic of nested pair-bias attention, on the CPU.

The geometry table the nested path builds is executed here by a small torch
interpreter of the table's addressing (element (g, h, i, d) of an operand at
``off + g*s_g + h*s_h + i*s_i + d``; mask ``off + g*s_g + i*s_q + key``), and
the result is compared with the per-sample dense oracle.  A wrong stride,
offset or packing order for any operand, mask or bias fails here without a
GPU.  Admission and error contracts are checked too.
"""

import pytest
import torch

from nested_pair_cases import LAYOUTS, expected_outputs, make_case
from nested_standin import NestedTensor
from oops_amd import OOpsUnsupportedError, _lib, pair_bias_attention
from oops_amd.attention import pair_bias_nested as pbn


def _view(t, off, size, stride):
    return torch.as_strided(t, size, stride, t.storage_offset() + off)


def _run_table(qv, kv, vv, mask_buf, bias_buf, table, heads, head_size, scale):
    out = torch.zeros_like(qv, dtype=torch.float64)
    W = _lib.TABLE_WIDTH
    for r in range(len(table) // W):
        row = table[r * W : (r + 1) * W]
        G, Lq, Lk = row[_lib.T_GROUPS], row[_lib.T_LEN_Q], row[_lib.T_LEN_K]

        def op(t, c):
            off, sg, sh, si = row[c : c + 4]
            return _view(t, off, (G, heads, Lq if c in (_lib.T_Q_OFF, _lib.T_O_OFF) else Lk, head_size), (sg, sh, si, 1))

        q, k, v = op(qv, _lib.T_Q_OFF).double(), op(kv, _lib.T_K_OFF).double(), op(vv, _lib.T_V_OFF).double()
        s = q @ k.transpose(-1, -2) * scale
        if row[_lib.T_B_OFF] >= 0 and bias_buf is not None:
            off, sg, sh, si = row[_lib.T_B_OFF : _lib.T_B_OFF + 4]
            s = s + _view(bias_buf, off, (G, heads, Lq, Lk), (sg, sh, si, 1)).double()
        if row[_lib.T_M_OFF] >= 0 and mask_buf is not None:
            off, sg, sq = row[_lib.T_M_OFF : _lib.T_M_OFF + 3]
            keep = _view(mask_buf, off, (G, 1, Lq, Lk), (sg, 0, sq, 1))
            s = s.masked_fill(~keep, float("-inf"))
        p = torch.softmax(s, -1).nan_to_num(0.0)
        o = p @ v
        off, sg, sh, si = row[_lib.T_O_OFF : _lib.T_O_OFF + 4]
        _view(out, off, (G, heads, Lq, head_size), (sg, sh, si, 1)).copy_(o)
    return out


def _plan(q, k, v, mask, bias):
    qo = pbn._operand("query", q)
    ko, vo = pbn._operand("key", k), pbn._operand("value", v)
    mask_buf, mask_cols = (None, None) if mask is None else pbn._mask_plan(mask, qo, ko)
    bias_buf, bias_cols, shared = (None, None, True) if bias is None else pbn._bias_plan(bias, qo, ko)
    table = pbn.plan_table(qo, ko, vo, mask_cols, bias_cols, shared)
    return qo, ko, vo, mask_buf, bias_buf, table


CASES = [
    ("implicit", "key", True, "full"),
    ("implicit", "pair", True, "shared_head"),
    ("static", "key", True, "shared"),
    ("static", "key", False, "full"),
    ("static", "pair", False, "shared_head"),
    ("static", "key_singleton", False, "shared"),
    ("group_outer", "key", False, "shared"),
    ("group_outer", "pair", True, "shared_head"),
    ("token_outer", "key", False, "shared"),
    ("token_outer", "key", True, "none"),
    ("ragged_groups", "key", False, "shared_head"),
    ("ragged_groups", "none", True, "shared"),
    ("ragged_groups_tokens", "key", False, "shared"),
]


@pytest.mark.parametrize("layout,mask_kind,mask_shared,bias_kind", CASES)
def test_table_addressing(layout, mask_kind, mask_shared, bias_kind):
    (q, k, v, mask, bias), _ = make_case(
        layout, dtype=torch.float64, mask_kind=mask_kind, mask_shared=mask_shared, bias_kind=bias_kind,
        groups=(2, 3) if layout != "static" else (3, 3), seed=len(layout),
    )  # fmt: skip
    qo, ko, vo, mask_buf, bias_buf, table = _plan(q, k, v, mask, bias)
    scale = 0.3
    out = _run_table(qo.values, ko.values, vo.values, mask_buf, bias_buf, table, qo.heads, qo.head_size, scale)
    got = q.packed_like(out.reshape(q.concat.shape)).unbind()
    want = expected_outputs(q, k, v, mask, bias, scale)
    assert len(got) == len(want)
    for g_, w_ in zip(got, want):
        torch.testing.assert_close(g_, torch.from_numpy(w_), atol=1e-10, rtol=1e-10)


def test_all_layouts_covered():
    assert {c[0] for c in CASES} == set(LAYOUTS)


def test_errors_on_cpu():
    (q, k, v, mask, bias), _ = make_case("static", mask_kind="key", bias_kind="shared")
    with pytest.raises(OOpsUnsupportedError):
        pair_bias_attention(q, k, v, mask, bias)  # CPU tensors are not served
    with pytest.raises(ValueError):
        pair_bias_attention(q, k.concat, v, mask, bias)
    with pytest.raises(ValueError):
        pair_bias_attention(q, k, v, mask.concat, bias)
    with pytest.raises(ValueError):
        pair_bias_attention(q, k, v, mask, bias.concat)
    with pytest.raises(ValueError):
        pair_bias_attention(q.concat, k.concat, v.concat, mask, None)
    # keys of one packing, queries of another
    (q2, _, _, _, _), _ = make_case("group_outer", mask_kind="none", bias_kind="none")
    with pytest.raises(ValueError):
        pair_bias_attention(q2, k, v)
    # key mask lengths that do not match K_i
    bad = NestedTensor([torch.ones(1, 3, dtype=torch.bool), torch.ones(1, 2, dtype=torch.bool)], ragged_dims=(1,))
    with pytest.raises(ValueError):
        pair_bias_attention(q, k, v, bad)
    # per-group bias over ragged groups is not served
    (qg, kg, vg, _, _), _ = make_case("group_outer", mask_kind="none", bias_kind="none")
    full = NestedTensor([torch.zeros(2, 2, 5, 7), torch.zeros(2, 2, 9, 4)], ragged_dims=(2, 3))
    with pytest.raises(OOpsUnsupportedError):
        pair_bias_attention(qg, kg, vg, None, full)
    # unsupported packing
    odd = NestedTensor(ragged_dims=(0,), packed_dim_order=(0, 1, 2), _sizes=[(5, 2, 16), (9, 2, 16)],
                       _concat=torch.zeros(14, 2, 16))  # fmt: skip
    with pytest.raises(OOpsUnsupportedError):
        pair_bias_attention(odd, odd, odd)
