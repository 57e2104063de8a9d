"""Nested (ragged MSA) pair-bias attention cases shared by the CPU and GPU tests.

Builds inputs the way the reference's ``_nested_inputs`` does
(tests/attention/pair_bias/test_pair_bias_attention.py:57-200) with the
DanLing stand-in, in every q/k/v packing the operator serves, and computes the
expected result by the reference's recipe (:203-226): unbind the samples, run
the dense oracle on each, and compare sample by sample.
"""

from __future__ import annotations

import numpy as np
import torch

from nested_standin import NestedTensor
from oracle import attention as ora

# layout -> (q/k/v element builder, ragged dims) ; see _qkv below
LAYOUTS = ("implicit", "static", "group_outer", "token_outer", "ragged_groups", "ragged_groups_tokens")


def _qkv_template(layout, groups, lengths, heads, head_size):
    if layout == "implicit":
        return NestedTensor([torch.empty(heads, n, head_size) for n in lengths], ragged_dims=(1,))
    if layout == "static":
        return NestedTensor([torch.empty(groups[0], heads, n, head_size) for n in lengths], ragged_dims=(2,))
    if layout == "group_outer":
        return NestedTensor([torch.empty(s, heads, n, head_size) for s, n in zip(groups, lengths)], ragged_dims=(0, 2))
    if layout == "token_outer":
        t = NestedTensor([torch.empty(n, heads, s, head_size) for s, n in zip(groups, lengths)], ragged_dims=(0, 2))
        return t.transpose(1, 3)
    if layout == "ragged_groups":
        return NestedTensor([torch.empty(s, heads, lengths[0], head_size) for s in groups], ragged_dims=(0,))
    if layout == "ragged_groups_tokens":  # (S_i, Q, H, D) packing, viewed as (S_i, H, Q, D)
        t = NestedTensor([torch.empty(s, lengths[0], heads, head_size) for s in groups], ragged_dims=(0,))
        return t.transpose(2, 3)
    raise ValueError(layout)


def make_case(layout, *, dtype=torch.float32, device="cpu", q_lengths=(5, 9), k_lengths=(7, 4), groups=(2, 3),
              heads=2, head_size=16, mask_kind="key", mask_shared=True, bias_kind="shared", seed=0,
              requires_grad=False):  # fmt: skip
    """Returns (query, key, value, mask, bias) nested inputs and the leaf value tensors."""

    g = torch.Generator().manual_seed(seed)
    grouped = layout in ("group_outer", "token_outer", "ragged_groups", "ragged_groups_tokens")
    if layout == "implicit":
        groups = (1,) * len(q_lengths)
    elif layout == "static":
        groups = (groups[0],) * len(q_lengths)
    if layout.startswith("ragged_groups"):
        q_lengths = (q_lengths[0],) * len(groups)
        k_lengths = (k_lengths[0],) * len(groups)
    n = len(groups)
    q_lengths, k_lengths = q_lengths[:n], k_lengths[:n]

    def values(tmpl):
        x = torch.randn(tmpl.concat.shape, generator=g).to(dtype).to(device)
        return tmpl.packed_like(x.requires_grad_(requires_grad)), x

    q, qv = values(_qkv_template(layout, groups, q_lengths, heads, head_size))
    k, kv = values(_qkv_template(layout, groups, k_lengths, heads, head_size))
    v, vv = values(_qkv_template(layout, groups, k_lengths, heads, head_size))

    mask = None
    if mask_kind != "none":
        if mask_kind == "key" and grouped and not mask_shared:
            # per-group key mask (S_i, 1, K_i) in the q/k/v packing
            if layout == "group_outer":
                tm = NestedTensor([torch.empty(s, 1, m, dtype=torch.bool) for s, m in zip(groups, k_lengths)],
                                  ragged_dims=(0, 2))  # fmt: skip
            elif layout == "token_outer":
                tm = NestedTensor([torch.empty(m, 1, s, dtype=torch.bool) for s, m in zip(groups, k_lengths)],
                                  ragged_dims=(0, 2)).transpose(1, 3)  # fmt: skip
            else:
                tm = NestedTensor([torch.empty(s, 1, k_lengths[0], dtype=torch.bool) for s in groups],
                                  ragged_dims=(0,))  # fmt: skip
        elif mask_kind == "key":
            if layout == "implicit":
                tm = NestedTensor([torch.empty(m, dtype=torch.bool) for m in k_lengths], ragged_dims=(0,))
            else:
                mg = 1 if mask_shared else groups[0]
                tm = NestedTensor([torch.empty(mg, m, dtype=torch.bool) for m in k_lengths], ragged_dims=(1,))
        elif mask_kind == "key_singleton":  # (S|1, 1, K_i) elements
            mg = 1 if mask_shared else groups[0]
            tm = NestedTensor([torch.empty(mg, 1, m, dtype=torch.bool) for m in k_lengths], ragged_dims=(2,))
        elif mask_kind == "pair":
            if layout == "implicit":
                tm = NestedTensor([torch.empty(a, m, dtype=torch.bool) for a, m in zip(q_lengths, k_lengths)],
                                  ragged_dims=(0, 1))  # fmt: skip
            else:
                mg = 1 if mask_shared else groups[0]
                tm = NestedTensor([torch.empty(mg, a, m, dtype=torch.bool) for a, m in zip(q_lengths, k_lengths)],
                                  ragged_dims=(1, 2))  # fmt: skip
        else:
            raise ValueError(mask_kind)
        mv = torch.rand(tm.concat.shape, generator=g) > 0.25
        mask = tm.packed_like(mv.to(device))

    bias = bv = None
    if bias_kind != "none":
        bh = 1 if bias_kind == "shared_head" else heads
        if layout == "implicit":
            tb = NestedTensor([torch.empty(bh, a, m) for a, m in zip(q_lengths, k_lengths)], ragged_dims=(1, 2))
        else:
            bg = groups[0] if bias_kind == "full" else 1
            tb = NestedTensor([torch.empty(bg, bh, a, m) for a, m in zip(q_lengths, k_lengths)], ragged_dims=(2, 3))
        bias, bv = values(tb)
    return (q, k, v, mask, bias), (qv, kv, vv, bv)


def _np(t):
    return None if t is None else t.detach().double().cpu().numpy()


def expected_outputs(q, k, v, mask, bias, scale=None):
    """Per-sample dense oracle (test_pair_bias_attention.py:203-213)."""

    parts = []
    masks = (None,) * len(q.unbind()) if mask is None else mask.unbind()
    biases = (None,) * len(q.unbind()) if bias is None else bias.unbind()
    for qe, ke, ve, me, be in zip(q.unbind(), k.unbind(), v.unbind(), masks, biases):
        parts.append(ora.pair_bias_attention_forward(_np(qe), _np(ke), _np(ve), _np(me), _np(be), scale))
    return parts


def expected_grads(q, k, v, mask, bias, douts, scale=None):
    """Per-sample oracle gradients packed back into each operand's packing."""

    masks = (None,) * len(douts) if mask is None else mask.unbind()
    biases = (None,) * len(douts) if bias is None else bias.unbind()
    dq, dk, dv, db = [], [], [], []
    for qe, ke, ve, me, be, de in zip(q.unbind(), k.unbind(), v.unbind(), masks, biases, douts):
        g = ora.pair_bias_attention_backward(_np(qe), _np(ke), _np(ve), _np(de), _np(me), _np(be), scale)
        for acc, x in zip((dq, dk, dv, db), g):
            acc.append(None if x is None else torch.from_numpy(np.ascontiguousarray(x)))

    def pack(nested, parts):
        return torch.cat([nested._pack(p) for p in parts])

    return pack(q, dq), pack(k, dk), pack(v, dv), (None if bias is None else pack(bias, db))
