"""CPU oracle for pair-biased attention — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker (or the timed CPU
baseline).  The product (``oops_amd``) never imports it and has no CPU path.

It restates, in numpy, the closed-form references the OOps tests compare
against:

* triangle attention: ``_reference`` in
  tests/attention/triangle/test_triangle_attention.py:42-58 — q/k/v
  ``(*prefix, R, C, H, D)`` are moved to ``(..., R, H, C, D)``;
  ``scores = (q @ k^T) * scale + bias``; masked keys get ``-inf``; rows with no
  kept key get all-zero logits; softmax; masked probabilities are zeroed;
  ``@ v``; moved back.
* MSA-row pair-bias attention: ``pair_bias_attention_reference`` in
  tests/references/pair_bias_attention.py:29-46 — head-major
  ``(*prefix, S, H, Q, D)``, a key mask ``(*, S, K)`` or pair mask
  ``(*, S, Q, K)``.

Gradients: the reference tests take them with autograd through the formula
(test_triangle_attention.py:344-370, :414); here the same derivative is written
out (softmax backward, flash-attention convention
oops/attention/flash/triton/kernel.py:53-62): P = softmax(S) with masked
entries 0, dP = dO V^T, delta = rowsum(dO * O), dS = P * (dP - delta),
dQ = scale dS K, dK = scale dS^T Q, dV = P^T dO, dBias = dS summed over the
broadcast axes of the bias.

Parity pins (tests/test_oracle.py): torch's scaled_dot_product_attention
(forward and autograd, with the bias as a float attn_mask), a pure-Python
brute-force loop, central finite differences of the forward, and the
invariants listed there.  The reference repository ships no golden vectors.

All work is chunked over rows so N=768 never materialises the full
``R x H x C x C`` score tensor.
"""

from __future__ import annotations

import math

import numpy as np


def _softmax_rows(scores: np.ndarray, keep: np.ndarray | None) -> np.ndarray:
    """Row softmax with the reference's mask convention (zero rows when nothing is kept)."""

    if keep is not None:
        any_keep = keep.any(axis=-1, keepdims=True)
        scores = np.where(keep, scores, -np.inf)
        scores = np.where(any_keep, scores, 0.0)
    m = scores.max(axis=-1, keepdims=True)
    e = np.exp(scores - m)
    p = e / e.sum(axis=-1, keepdims=True)
    if keep is not None:
        p = np.where(keep, p, 0.0)
    return p


def _row_chunk(rows: int, cols: int, heads: int, budget: int = 1 << 25) -> int:
    per_row = max(1, heads * cols * cols)
    return max(1, min(rows, budget // per_row))


def triangle_attention_forward(q, k, v, mask=None, bias=None, scale=None, *, dtype=np.float64):
    """Forward of triangle attention; returns (out, lse) with lse ``(*prefix, R, H, C)`` (natural log).

    Follows tests/attention/triangle/test_triangle_attention.py:42-58.
    """

    q, k, v = (np.asarray(x, dtype=dtype) for x in (q, k, v))
    *prefix, R, C, H, D = q.shape
    scale = D**-0.5 if scale is None else scale
    qh, kh, vh = (np.swapaxes(x, -2, -3) for x in (q, k, v))  # (..., R, H, C, D)
    keep_full = None
    if mask is not None:
        keep_full = np.broadcast_to(np.asarray(mask, dtype=bool), (*prefix, R, C))
    b = None if bias is None else np.asarray(bias, dtype=dtype)
    if keep_full is not None:
        # masked keys read K/V as zero (reference kernel.py:220-223), so
        # non-finite values behind the mask never reach the output
        kh, vh = _zero_masked_keys(kh, vh, keep_full)
    out = np.empty(qh.shape, dtype=dtype)
    lse = np.empty((*prefix, R, H, C), dtype=dtype)
    step = _row_chunk(R, C, H)
    for r0 in range(0, R, step):
        sl = slice(r0, min(R, r0 + step))
        s = np.matmul(qh[..., sl, :, :, :], np.swapaxes(kh[..., sl, :, :, :], -1, -2)) * scale
        if b is not None:
            bb = b[..., sl, :, :, :] if b.shape[-4] != 1 else b
            s = s + bb
        keep = None if keep_full is None else keep_full[..., sl, None, None, :]
        if keep is not None:
            keep = np.broadcast_to(keep, s.shape)
        p = _softmax_rows(s, keep)
        out[..., sl, :, :, :] = np.matmul(p, vh[..., sl, :, :, :])
        if keep is None:
            masked = s
        else:
            masked = np.where(keep, s, -np.inf)
        mx = masked.max(axis=-1)
        with np.errstate(invalid="ignore", divide="ignore"):
            l = np.log(np.exp(masked - np.where(np.isfinite(mx), mx, 0.0)[..., None]).sum(axis=-1))
            lse[..., sl, :, :] = np.where(np.isfinite(mx), mx + l, 0.0)
    return np.swapaxes(out, -2, -3), lse


def triangle_attention_backward(q, k, v, dout, mask=None, bias=None, scale=None, *, dtype=np.float64):
    """Gradients (dq, dk, dv, dbias) of ``sum(out * dout)``; dbias has the bias's shape."""

    q, k, v, dout = (np.asarray(x, dtype=dtype) for x in (q, k, v, dout))
    *prefix, R, C, H, D = q.shape
    scale = D**-0.5 if scale is None else scale
    qh, kh, vh, doh = (np.swapaxes(x, -2, -3) for x in (q, k, v, dout))
    keep_full = None
    if mask is not None:
        keep_full = np.broadcast_to(np.asarray(mask, dtype=bool), (*prefix, R, C))
    b = None if bias is None else np.asarray(bias, dtype=dtype)
    shared = b is not None and b.shape[-4] == 1
    if keep_full is not None:
        kh, vh = _zero_masked_keys(kh, vh, keep_full)
    dq = np.empty(qh.shape, dtype=dtype)
    dk = np.empty(kh.shape, dtype=dtype)
    dv = np.empty(vh.shape, dtype=dtype)
    # dS accumulates at the full prefix; axes the bias broadcasts over are summed at the end
    db = None if b is None else np.zeros((*prefix, *b.shape[-4:]), dtype=dtype)
    step = _row_chunk(R, C, H)
    for r0 in range(0, R, step):
        sl = slice(r0, min(R, r0 + step))
        qs, ks, vs, dos = (x[..., sl, :, :, :] for x in (qh, kh, vh, doh))
        s = np.matmul(qs, np.swapaxes(ks, -1, -2)) * scale
        if b is not None:
            s = s + (b if shared else b[..., sl, :, :, :])
        keep = None if keep_full is None else np.broadcast_to(keep_full[..., sl, None, None, :], s.shape)
        p = _softmax_rows(s, keep)
        o = np.matmul(p, vs)
        dp = np.matmul(dos, np.swapaxes(vs, -1, -2))
        delta = (dos * o).sum(axis=-1, keepdims=True)
        ds = p * (dp - delta)
        dq[..., sl, :, :, :] = np.matmul(ds, ks) * scale
        dk[..., sl, :, :, :] = np.matmul(np.swapaxes(ds, -1, -2), qs) * scale
        dv[..., sl, :, :, :] = np.matmul(np.swapaxes(p, -1, -2), dos)
        if db is not None:
            if shared:
                db += ds.sum(axis=-4, keepdims=True)
            else:
                db[..., sl, :, :, :] = ds
    if db is not None:
        lead = db.ndim - b.ndim
        db = db.sum(axis=tuple(range(lead))) if lead else db
        for axis, size in enumerate(b.shape[:-4]):
            if size == 1 and db.shape[axis] != 1:
                db = db.sum(axis=axis, keepdims=True)
    if keep_full is not None:
        key_keep = keep_full[..., None, :, None]  # (..., R, 1, C, 1) against (..., R, H, C, D)
        dk = np.where(key_keep, dk, 0.0)
        dv = np.where(key_keep, dv, 0.0)
    return (np.swapaxes(dq, -2, -3), np.swapaxes(dk, -2, -3), np.swapaxes(dv, -2, -3), db)


def _zero_masked_keys(kh, vh, keep):
    key_keep = keep[..., None, :, None]
    return np.where(key_keep, kh, 0.0), np.where(key_keep, vh, 0.0)


def triangle_attention_bruteforce(q, k, v, mask=None, bias=None, scale=None):
    """Pure-Python loop version of the forward for tiny shapes (index/transposition check)."""

    q, k, v = (np.asarray(x, dtype=np.float64) for x in (q, k, v))
    *prefix, R, C, H, D = q.shape
    scale = D**-0.5 if scale is None else scale
    qf = q.reshape(-1, R, C, H, D)
    kf = k.reshape(-1, R, C, H, D)
    vf = v.reshape(-1, R, C, H, D)
    B = qf.shape[0]
    keep = None if mask is None else np.broadcast_to(np.asarray(mask, bool), (*prefix, R, C)).reshape(B, R, C)
    bf = None if bias is None else np.asarray(bias, np.float64).reshape(B, -1, H, C, C)
    out = np.zeros_like(qf)
    for bi in range(B):
        for r in range(R):
            for h in range(H):
                for i in range(C):
                    kept = [j for j in range(C) if keep is None or keep[bi, r, j]]
                    if not kept:
                        continue
                    logits = []
                    for j in kept:
                        s = sum(qf[bi, r, i, h, d] * kf[bi, r, j, h, d] for d in range(D)) * scale
                        if bf is not None:
                            s += bf[bi, 0 if bf.shape[1] == 1 else r, h, i, j]
                        logits.append(s)
                    m = max(logits)
                    w = [math.exp(x - m) for x in logits]
                    z = sum(w)
                    for d in range(D):
                        out[bi, r, i, h, d] = sum(wj * vf[bi, r, j, h, d] for wj, j in zip(w, kept)) / z
    return out.reshape(q.shape)


# ------------------------------------------------------------------ MSA row pair-bias attention


def _pair_keep(mask, q_shape, k_len):
    """Broadcastable keep tensor for head-major scores ``(*, S, H, Q, K)``.

    Follows tests/references/pair_bias_attention.py:37-43: a mask with rank
    ``q.dim() - 2`` is a key mask ``(*, S, K)``; otherwise a pair mask
    ``(*, S, Q, K)`` (optionally with a unit head axis).
    """

    if mask is None:
        return None
    keep = np.asarray(mask, dtype=bool)
    if keep.ndim == len(q_shape) - 2:
        keep = keep[..., None, None, :]
    else:
        while keep.ndim < len(q_shape):
            keep = keep[..., None, :, :] if keep.ndim == len(q_shape) - 1 else keep[None]
    return keep


def pair_bias_attention_forward(q, k, v, mask=None, bias=None, scale=None, *, dtype=np.float64):
    """Forward of head-major pair-bias attention ``(*prefix, S, H, Q, D)``."""

    q, k, v = (np.asarray(x, dtype=dtype) for x in (q, k, v))
    D = q.shape[-1]
    scale = D**-0.5 if scale is None else scale
    s = np.matmul(q, np.swapaxes(k, -1, -2)) * scale
    if bias is not None:
        s = s + np.asarray(bias, dtype=dtype)
    keep = _pair_keep(mask, q.shape, k.shape[-2])
    if keep is not None:
        keep = np.broadcast_to(keep, s.shape)
    p = _softmax_rows(s, keep)
    return np.matmul(p, v)


def pair_bias_attention_backward(q, k, v, dout, mask=None, bias=None, scale=None, *, dtype=np.float64):
    """(dq, dk, dv, dbias) of ``sum(out * dout)``; dbias summed to the bias's shape."""

    q, k, v, dout = (np.asarray(x, dtype=dtype) for x in (q, k, v, dout))
    D = q.shape[-1]
    scale = D**-0.5 if scale is None else scale
    s = np.matmul(q, np.swapaxes(k, -1, -2)) * scale
    b = None if bias is None else np.asarray(bias, dtype=dtype)
    if b is not None:
        s = s + b
    keep = _pair_keep(mask, q.shape, k.shape[-2])
    if keep is not None:
        keep = np.broadcast_to(keep, s.shape)
    p = _softmax_rows(s, keep)
    o = np.matmul(p, v)
    dp = np.matmul(dout, np.swapaxes(v, -1, -2))
    ds = p * (dp - (dout * o).sum(axis=-1, keepdims=True))
    dq = np.matmul(ds, k) * scale
    dk = np.matmul(np.swapaxes(ds, -1, -2), q) * scale
    dv = np.matmul(np.swapaxes(p, -1, -2), dout)
    db = None
    if b is not None:
        db = ds
        # sum over leading axes the bias lacks, then over its unit axes
        while db.ndim > b.ndim:
            db = db.sum(axis=0)
        for axis, size in enumerate(b.shape):
            if size == 1 and db.shape[axis] != 1:
                db = db.sum(axis=axis, keepdims=True)
    return dq, dk, dv, db


def shared_dbias_at(q, k, v, dout, mask=None, bias=None, qpos=None, scale=None, *, rows_per_chunk=32,
                    dtype=np.float64):
    """Row-shared dBias ``(H, len(qpos), K)`` of head-major pair-bias attention ``(S, H, Q, D)`` at the
    query positions ``qpos`` (all when None), summed over all S rows, chunked over rows.

    Queries are independent (each is one softmax over the keys), so restricting them is exact: this is
    ``pair_bias_attention_backward(...)[3][0][:, qpos]`` at a fraction of its memory.  ``mask`` is a
    key mask ``(S, K)`` or None; ``bias`` is ``(1, H, Q, K)``.
    """

    S, H, Q, D = np.shape(q)
    qpos = np.arange(Q) if qpos is None else np.asarray(qpos)
    b = None if bias is None else np.asarray(bias)[:, :, qpos]
    acc = np.zeros((H, len(qpos), np.shape(k)[-2]), dtype=dtype)
    for r0 in range(0, S, rows_per_chunk):
        sl = slice(r0, min(S, r0 + rows_per_chunk))
        m = None if mask is None else np.asarray(mask)[sl]
        *_, db = pair_bias_attention_backward(np.asarray(q)[sl][:, :, qpos], np.asarray(k)[sl], np.asarray(v)[sl],
                                              np.asarray(dout)[sl][:, :, qpos], m, b, scale, dtype=dtype)
        acc += db[0]
    return acc
