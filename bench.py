"""Headline benchmark: triangle attention (ending node) fwd+bwd, N=768, H=4, c=32, bf16, one MI355X.

One "step" = forward + backward (dQ, dK, dV, dBias) of ``oops_amd.triangle_attention`` on
q, k, v ``randn(1, 768, 768, 4, 32)`` bf16 passed as ``.transpose(1, 2)``
views (ending node, swapped pair axes, read in place), bias ``randn(1, 1, 4, 768, 768)`` bf16
shared over rows, no mask, upstream gradient ``randn`` in the output's layout.  Inputs are
resident in HBM before timing.  Algorithmic FLOPs per step = 14 * H * c * N^3 (the flash
attention convention: seven N x N x c products per row and head, two forward (QK^T, PV) and five
backward (QK^T again, dO V^T, P^T dO, dS K, dS^T Q), 2 * H * c * N^3 each).

Prints ONE JSON line with the driver's contract fields plus ``roofline`` (dominant kernel,
timed live with HIP events on the launch stream) and ``cpu_baseline`` (the numpy oracle on
a bounded row sample, on this host's cores).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "tri-attn fwd+bwd TFLOP/s & ms/call at N=768 bf16; MFMA util % vs peak"
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0
PEAK_F32_TFLOPS = 157.3  # MI355X dense fp32 MFMA
COPY_CAL_BYTES = 256 << 20
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "triangle_attention_c3_bf16_traffic.txt")
MFMA_FILE = os.path.join(ROOT, "profiles", "triangle_attention_c3_bf16_mfma.txt")
N, H, C = 768, 4, 32


def flops_step(n=N, h=H, c=C):
    return 14 * h * c * n**3


def _log(msg):
    print(msg, file=sys.stderr, flush=True)


def make_inputs(device, seed=2):
    import torch

    g = torch.Generator(device="cpu").manual_seed(seed)
    base = [torch.randn(1, N, N, H, C, generator=g).to(torch.bfloat16).to(device) for _ in range(3)]
    q, k, v = (b.transpose(1, 2).requires_grad_(True) for b in base)
    bias = torch.randn(1, 1, H, N, N, generator=g).to(torch.bfloat16).to(device).requires_grad_(True)
    # upstream gradient in the output's (ending-node) layout
    dout = torch.randn(1, N, N, H, C, generator=g).to(torch.bfloat16).to(device).transpose(1, 2)
    return q, k, v, bias, dout


def step(q, k, v, bias, dout):
    import torch

    from oops_amd import triangle_attention

    out = triangle_attention(q, k, v, None, bias)
    return torch.autograd.grad(out, (q, k, v, bias), dout)


def time_events(fn, iters, warmup, stream):
    import torch

    for _ in range(warmup):
        fn()
    times = []
    for _ in range(iters):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        fn()
        b.record(stream)
        b.synchronize()
        times.append(a.elapsed_time(b))
    return statistics.median(times)


def time_events_batched(fn, iters, warmup, stream, batch=10):
    """Median ms per call of `batch` back-to-back calls between one event pair: the host enqueues the
    next call while the GPU runs the current one, so host-side work between calls is not counted."""

    import torch

    for _ in range(warmup):
        fn()
    times = []
    for _ in range(iters):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(batch):
            fn()
        b.record(stream)
        b.synchronize()
        times.append(a.elapsed_time(b) / batch)
    return statistics.median(times)


def kernel_times(q, k, v, bias, dout, iters=20):
    """Median ms of each kernel, each launched alone on the current stream (HIP events)."""

    import torch

    from oops_amd import _lib
    from oops_amd.attention import _core

    stream = torch.cuda.current_stream()
    out = triangle_attention_out = None
    from oops_amd import triangle_attention

    with torch.no_grad():
        out = triangle_attention(q, k, v, None, bias)
    # rebuild the op-level arguments exactly as the front-end does
    qd, kd, vd, bd = (t.detach() for t in (q, k, v, bias))
    table = []
    for _ in range(1):
        table += _core.table_row(
            groups=N, len_q=N, len_k=N,
            q=(0, qd.stride(1), qd.stride(3), qd.stride(2)),
            k=(0, kd.stride(1), kd.stride(3), kd.stride(2)),
            v=(0, vd.stride(1), vd.stride(3), vd.stride(2)),
            bias=(0, 0, bd.stride(2), bd.stride(3)), dbias=(0, 0, N * N, N), bias_mode=_lib.BIAS_SHARED,
            lse_off=0,
        )  # fmt: skip
    scale = C**-0.5
    lse_numel = N * H * N
    fwd = lambda: _core.attention_forward(qd, kd, vd, None, bd, table, H, scale, lse_numel, True)
    o, o_lo, lse = fwd()
    res = {"fwd": time_events(fwd, iters, 3, stream)}
    # dq includes delta = rowsum(O * dO), which the dQ kernel computes itself; dkvb is the fused
    # dK/dV + shared-dBias kernel with the reduction of its per-part dBias slabs
    for name, ph in (("dq", _lib.PHASE_DQ), ("dkvb", _lib.PHASE_DKV | _lib.PHASE_DBIAS)):

        def bwd(ph=ph):
            with _core.profile_phases(ph):
                _core.attention_backward(dout, qd, kd, vd, None, bd, o, o_lo, lse, table, H, scale, bd.numel(),
                                         [True, True, True, True])  # fmt: skip

        res[name] = time_events(bwd, iters, 3, stream)
    # the isolated backward call also allocates outputs/workspace; measure that overhead with no kernels
    def empty_bwd():
        with _core.profile_phases(0x10):
            _core.attention_backward(dout, qd, kd, vd, None, bd, o, o_lo, lse, table, H, scale, bd.numel(),
                                     [True, True, True, True])  # fmt: skip

    overhead = time_events(empty_bwd, iters, 3, stream)
    for name in ("dq", "dkvb"):
        res[name] = max(res[name] - overhead, 1e-6)
    return res


def measured_traffic(kernel):
    """HBM bytes per dispatch of ``kernel`` from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
    summary (raw KiB readings scaled by a plain copy's readings), or None if absent."""

    try:
        lines = open(TRAFFIC_FILE).read().splitlines()
    except OSError:
        return None
    factors, rows = {}, {}
    for ln in lines:
        parts = ln.split()
        if not parts or ln.startswith("#"):
            continue
        if len(parts) == 2:
            factors[parts[0]] = float(parts[1])
        elif len(parts) == 3:
            rows[parts[0]] = (float(parts[1]), float(parts[2]))
    if kernel not in rows:
        return None
    fetch, write = rows[kernel]
    return int((fetch * factors.get("fetch_factor", 1.0) + write * factors.get("write_factor", 1.0)) * 1024)


def measured_mfma():
    """Per-kernel MFMA busy % from the committed rocprofv3 counter summary (SQ_VALU_MFMA_BUSY_CYCLES
    over every SIMD's cycles), or {} if absent."""

    out = {}
    try:
        lines = open(MFMA_FILE).read().splitlines()
    except OSError:
        return out
    for ln in lines:
        parts = ln.split()
        if len(parts) >= 2 and not ln.startswith("#"):
            out[parts[0]] = float(parts[1])
    return out


def accuracy(q, k, v, bias, dout):
    """Max-abs and mean-relative error of this step's outputs against the float64 oracle (the checker,
    never the thing measured): O, dQ, dK, dV on rows 0, 257, 511, 767; the shared dBias, which sums
    over all 768 rows, on 96 query positions (a 1-in-8 stride with a rotating offset, so every 32-query
    tile is covered) of every head and key.  dBias is reported twice: as returned (bf16) and as the
    kernels' float32 sums before that cast, with the error in bf16 ulps of the oracle's value."""

    import numpy as np
    import torch

    from oops_amd import triangle_attention
    from oops_amd.attention import _core
    from oracle import attention as ora

    with _core.capture_dbias_f32() as cap:
        out = triangle_attention(q, k, v, None, bias)
        grads = torch.autograd.grad(out, (q, k, v, bias), dout)
    db32 = cap.values[0][0, 0]
    npy = lambda t: t.detach().double().cpu().numpy()
    qn, kn, vn, don, bn = (npy(t) for t in (q, k, v, dout, bias))
    rows = [0, 257, 511, 767]
    o_want, _ = ora.triangle_attention_forward(qn[:, rows], kn[:, rows], vn[:, rows], None, bn)
    g_want = ora.triangle_attention_backward(qn[:, rows], kn[:, rows], vn[:, rows], don[:, rows], None, bn)
    qpos = [8 * j + (3 * j) % 8 for j in range(N // 8)]
    hm = lambda x: np.swapaxes(x[0].astype(np.float32), 1, 2)  # (rows, cols, H, D) -> (rows, H, cols, D)
    db_want = ora.shared_dbias_at(hm(qn), hm(kn), hm(vn), hm(don), None, bn[0], qpos)
    res = {"reference": "float64 numpy oracle", "tolerance": "bf16: |err| / max(1, |ref|) <= 2e-2",
           "dbias_queries": f"{len(qpos)} of {N} (every 32-query tile), all heads, all keys, summed over all rows"}
    pairs = (("out", out[:, rows], o_want), ("dq", grads[0][:, rows], g_want[0]), ("dk", grads[1][:, rows], g_want[1]),
             ("dv", grads[2][:, rows], g_want[2]), ("dbias", grads[3][0, 0][:, qpos], db_want),
             ("dbias_f32_precast", db32[:, qpos], db_want))
    for name, got, want in pairs:
        err = np.abs(npy(got) - want)
        at = np.unravel_index(err.argmax(), err.shape)
        res[name] = {"max_abs": float(f"{err.max():.4g}"),
                     "ref_at_max_abs": float(f"{want[at]:.4g}"),
                     "mean_rel": float(f"{err.mean() / max(np.abs(want).mean(), 1e-30):.4g}"),
                     "max_scaled": float(f"{(err / np.maximum(1.0, np.abs(want))).max():.4g}")}
        if name.startswith("dbias"):
            # in bf16 ulps of the oracle value, 2^(floor(log2 |ref|) - 7), where |ref| >= 1 (below that the
            # criterion is absolute and an ulp of a near-zero value says nothing)
            big = np.abs(want) >= 1.0
            ulp = np.exp2(np.floor(np.log2(np.abs(want[big]))) - 7)
            res[name]["max_err_bf16_ulps_ref_ge_1"] = float(f"{(err[big] / ulp).max():.3g}")
    return res


# per-kernel MFMA work in units of 2*H*c*N^3 (one N x N x c GEMM per row and head)
KERNEL_GEMMS = {"fwd": 2, "dq": 3, "dkvb": 4}


def bias_traffic(kt):
    """Bias bytes per kernel at config 3 (no mask there): each kernel reads the shared [H, N, N] bf16 bias
    (its fragment-major copy) from HBM once and re-reads it from L2 for every one of the N rows.  Rates are
    those bytes over the kernel's measured time."""

    once = H * N * N * 2
    reuse = {"fwd": N, "dq": N, "dkvb": N}
    out = {"bias_bytes": once, "mask_bytes": 0}
    for k, ms in kt.items():
        out[k] = {
            "hbm_gbps": round(once / (ms * 1e-3) / 1e9, 1),
            "l2_gbps": round(reuse.get(k, 1) * once / (ms * 1e-3) / 1e9, 1),
        }
    return out


def _median_ms(fn, iters=10, warmup=3, reps=3):
    """ms per call of `iters` back-to-back calls (median of `reps` runs): the
    host enqueues while the GPU works, as in a training loop."""

    import torch

    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        fn()
    runs = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(stream)
        for _ in range(iters):
            fn()
        b.record(stream)
        b.synchronize()
        runs.append(a.elapsed_time(b) / iters)
    return statistics.median(runs)


def other_configs(device, which=("c2", "c4", "c5")):
    """fwd+bwd ms and TFLOP/s of BASELINE configs 2, 4 and 5 (parity cases, reported beside the headline);
    ``which`` selects a subset (one config per profiler run keeps their kernel statistics apart)."""

    import torch

    from oops_amd import pair_bias_attention, triangle_attention

    res = {}

    def grad_step(fn, leaves, dout):
        def run():
            out = fn()
            o = out.concat if hasattr(out, "concat") else out
            torch.autograd.grad(o, leaves, dout)

        return run

    # C2: starting node, N=384, key padding of the last 10-30% (seed 1)
    if "c2" in which:
        res.update(_config2(device, grad_step))
    if "c4" in which:
        res.update(_config4(device, grad_step))
    if "c5" in which:
        res.update(_config5(device, grad_step))
    return res


def _config2(device, grad_step):
    import torch

    from oops_amd import triangle_attention

    res = {}
    g = torch.Generator().manual_seed(1)
    n = 384
    q, k, v, do = (torch.randn(1, n, n, H, C, generator=g).to(torch.bfloat16).to(device) for _ in range(4))
    bias = torch.randn(1, 1, H, n, n, generator=g).to(torch.bfloat16).to(device)
    keep = n - round(n * float(torch.empty(1).uniform_(0.10, 0.30, generator=g)))
    mask = torch.ones(1, n, n, dtype=torch.bool, device=device)
    mask[..., keep:] = False
    mask[:, keep:, :] = False
    leaves = [t.requires_grad_(True) for t in (q, k, v, bias)]
    ms = _median_ms(grad_step(lambda: triangle_attention(q, k, v, mask, bias), leaves, do))
    res["c2_starting_n384_keypad"] = {"ms": round(ms, 4), "tflops": round(14 * H * C * n**3 / ms / 1e9, 2)}
    return res


def _config4(device, grad_step):
    import torch

    from oops_amd import pair_bias_attention

    res = {}
    # C4: MSA rows S=512, N=384, H=8 head-major, key mask ~15%, shared bias (seed 3)
    g = torch.Generator().manual_seed(3)
    s_, n, h = 512, 384, 8
    q, k, v = (torch.randn(s_, n, h, C, generator=g).to(torch.bfloat16).permute(0, 2, 1, 3).to(device)
               for _ in range(3))  # fmt: skip
    bias = torch.randn(1, h, n, n, generator=g).to(torch.bfloat16).to(device)
    mask = torch.rand(s_, n, generator=g) > 0.15
    mask[:, 0] = True
    mask = mask.to(device)
    do = torch.randn(s_, h, n, C, generator=g).to(torch.bfloat16).to(device)
    leaves = [t.requires_grad_(True) for t in (q, k, v, bias)]
    ms = _median_ms(grad_step(lambda: pair_bias_attention(q, k, v, mask, bias), leaves, do))
    res["c4_msa_rows_s512_n384_h8"] = {"ms": round(ms, 4), "tflops": round(14 * s_ * h * C * n**2 / ms / 1e9, 2)}
    return res


def _config5(device, grad_step):
    import torch

    from oops_amd import triangle_attention

    res = {}
    # C5: ragged complexes N_i in {256, 512, 768, 1024}, both orientations, key masks hiding 0-20% (seed 4)
    tests_dir = os.path.join(ROOT, "tests")
    if tests_dir not in sys.path:
        sys.path.insert(0, tests_dir)
    from nested_standin import NestedTensor  # DanLing's NestedTensor is not installed here

    g = torch.Generator().manual_seed(4)
    lengths = (256, 512, 768, 1024)
    tmpl = NestedTensor([torch.empty(n_, n_, H, C) for n_ in lengths], ragged_dims=(0, 1))
    vals = [torch.randn(tmpl.concat.shape, generator=g).to(torch.bfloat16).to(device).requires_grad_(True)
            for _ in range(3)]  # fmt: skip
    btmpl = NestedTensor([torch.empty(1, H, n_, n_) for n_ in lengths], ragged_dims=(2, 3))
    bvals = torch.randn(btmpl.concat.shape, generator=g).to(torch.bfloat16).to(device).requires_grad_(True)
    masks = []
    for n_ in lengths:
        hide = int(n_ * 0.2 * float(torch.rand(1, generator=g)))
        m = torch.ones(n_, n_, dtype=torch.bool)
        if hide:
            m[:, n_ - hide :] = False
        masks.append(m)
    mtmpl = NestedTensor(masks, ragged_dims=(0, 1))
    nmask = mtmpl.packed_like(mtmpl.concat.to(device))
    nq, nk, nv = (tmpl.packed_like(x) for x in vals)
    nb = btmpl.packed_like(bvals)
    tq, tk, tv = (t.transpose(-4, -3) for t in (nq, nk, nv))
    tm, tb = nmask.transpose(-2, -1), nb.transpose(-2, -1)
    dvals = torch.randn(tmpl.concat.shape, generator=g).to(torch.bfloat16).to(device)
    leaves = [*vals, bvals]

    def both():
        o1 = triangle_attention(nq, nk, nv, nmask, nb).concat
        o2 = triangle_attention(tq, tk, tv, tm, tb).concat
        torch.autograd.grad((o1, o2), leaves, (dvals, dvals))

    ms = _median_ms(both, iters=5, warmup=2)
    flops = 2 * 14 * H * C * sum(n_**3 for n_ in lengths)
    res["c5_ragged_both_directions"] = {"ms": round(ms, 4), "tflops": round(flops / ms / 1e9, 2)}
    return res


def nested_msa(device):
    """Ragged MSA pair-bias attention (the nested row after the headline path): samples with
    (S_i, N_i) = (256, 384), (128, 256), (128, 512), H=8, c=32, bf16, group-outer packing
    (elements (S_i, H, N_i, c)), a per-sequence key mask hiding ~15%, a shared pair bias per sample;
    fwd+bwd of every operand.  Comparable with config 4's dense MSA rows."""

    import torch

    from oops_amd import pair_bias_attention

    tests_dir = os.path.join(ROOT, "tests")
    if tests_dir not in sys.path:
        sys.path.insert(0, tests_dir)
    from nested_standin import NestedTensor  # DanLing's NestedTensor is not installed here

    g = torch.Generator().manual_seed(6)
    shapes = ((256, 384), (128, 256), (128, 512))
    h = 8
    tmpl = NestedTensor([torch.empty(s_, h, n_, C) for s_, n_ in shapes], ragged_dims=(0, 2))
    vals = [torch.randn(tmpl.concat.shape, generator=g).to(torch.bfloat16).to(device).requires_grad_(True)
            for _ in range(3)]  # fmt: skip
    btmpl = NestedTensor([torch.empty(1, h, n_, n_) for _, n_ in shapes], ragged_dims=(2, 3))
    bvals = torch.randn(btmpl.concat.shape, generator=g).to(torch.bfloat16).to(device).requires_grad_(True)
    mtmpl = NestedTensor([torch.empty(s_, 1, n_, dtype=torch.bool) for s_, n_ in shapes], ragged_dims=(0, 2))
    mvals = torch.rand(mtmpl.concat.shape, generator=g) > 0.15
    mask = mtmpl.packed_like(mvals.to(device))
    q, k, v = (tmpl.packed_like(x) for x in vals)
    bias = btmpl.packed_like(bvals)
    dvals = torch.randn(tmpl.concat.shape, generator=g).to(torch.bfloat16).to(device)
    leaves = [*vals, bvals]

    def run():
        out = pair_bias_attention(q, k, v, mask, bias).concat
        torch.autograd.grad(out, leaves, dvals)

    ms = _median_ms(run, iters=10, warmup=3)
    flops = 14 * h * C * sum(s_ * n_**2 for s_, n_ in shapes)
    return {
        "workload": "nested pair_bias_attention fwd+bwd, (S_i, N_i) = (256,384),(128,256),(128,512), H=8, c=32, bf16",
        "ms_fwd_bwd": round(ms, 4),
        "tflops": round(flops / ms / 1e9, 2),
    }


def trimul_stage(device, n=512, c=128, h=128, dtype="bf16"):
    """triangle_multiplication (outgoing) fwd+bwd on one (N, N, C) pair, C = H = 128, bf16 (or float32), a
    key-padding style mask, projection biases; the row after attention in the Pairformer block.  Reports
    the whole fwd+bwd and the algorithmic GEMM rate (projections, contraction, output)."""

    import torch

    from oops_amd import triangle_multiplication

    g = torch.Generator().manual_seed(13)
    dt = {"bf16": torch.bfloat16, "f32": torch.float32}[dtype]

    def r(*shape, scale=1.0):
        return (torch.randn(*shape, generator=g) * scale).to(dt).to(device).requires_grad_(True)

    pair = r(1, n, n, c)
    mask = torch.ones(1, n, n, device=device)
    mask[:, :, n - n // 8 :] = 0
    mask[:, n - n // 8 :, :] = 0
    w = dict(
        input_norm_weight=r(c), input_norm_bias=r(c),
        left_value_weight=r(h, c, scale=c**-0.5), left_gate_weight=r(h, c, scale=c**-0.5),
        right_value_weight=r(h, c, scale=c**-0.5), right_gate_weight=r(h, c, scale=c**-0.5),
        output_norm_weight=r(h), output_norm_bias=r(h),
        output_weight=r(c, h, scale=h**-0.5), output_gate_weight=r(c, c, scale=c**-0.5),
        left_value_bias=r(h), left_gate_bias=r(h), right_value_bias=r(h), right_gate_bias=r(h),
        output_bias=r(c), output_gate_bias=r(c),
    )  # fmt: skip
    leaves = [pair, *w.values()]
    dy = torch.randn(1, n, n, c, generator=g).to(dt).to(device)

    def fwd():
        return triangle_multiplication(pair, mask, direction="outgoing", **w)

    def step():
        torch.autograd.grad(fwd(), leaves, dy)

    ms = _median_ms(step, iters=10, warmup=3)
    with torch.no_grad():
        ms_fwd = _median_ms(fwd, iters=10, warmup=3)
    rows = n * n
    fwd_flops = 2 * rows * c * 4 * h + 2 * h * n**3 + 2 * rows * (h + c) * c
    flops = 3 * fwd_flops  # backward: two products per forward product

    # the factor projection kernels alone (the largest HIP kernels of the update), through the C ABI on
    # the operator's own prepared operands, against HBM: forward reads xn and writes both factors,
    # backward also reads the factor gradients and writes the [4H][R] projection gradients
    import ctypes
    import importlib

    from oops_amd import _lib

    tm = importlib.import_module("oops_amd.pair.triangle_multiplication")
    lib = _lib.load()
    with torch.no_grad():
        grouped = pair.detach().reshape(1, rows, c)
        ops = tm._prepare(grouped, mask.reshape(1, rows), tuple(list(w.values())[:10]), tuple(list(w.values())[10:]))
        _pair, mask32, w_cat = ops[:3]
        b_cat = tm._small_views(ops[5], ops[6])[0]
        saved = tm.trimul_forward(*ops, [0, n], "outgoing", 1e-5, 1e-5)
        xn, factors = saved[1], saved[4]
        geo = tm._geometry(grouped, h, True, 1e-5)
        stream = torch.cuda.current_stream().cuda_stream
        d_fac = torch.randn_like(factors)
        d_proj = torch.empty(4 * h, rows, dtype=dt, device=device)
        bparts = torch.empty(lib.oops_trimul_bias_parts(ctypes.byref(geo)), 4 * h, device=device)
        ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731

        def f_fwd():
            lib.oops_trimul_factors_forward(ctypes.byref(geo), ptr(xn), ptr(w_cat), ptr(b_cat), ptr(mask32),
                                            ptr(factors), stream)  # fmt: skip

        def f_bwd():
            lib.oops_trimul_factors_backward(ctypes.byref(geo), ptr(xn), ptr(w_cat), ptr(b_cat), ptr(mask32),
                                             ptr(d_fac), ptr(d_proj), None, ptr(bparts), stream)  # fmt: skip

        k_fwd = _median_ms(f_fwd, iters=20, warmup=3)
        k_bwd = _median_ms(f_bwd, iters=20, warmup=3)
    el = 2 if dtype == "bf16" else 4
    fwd_bytes = rows * c * el + 2 * h * rows * el
    bwd_bytes = rows * c * el + 2 * h * rows * el + 4 * h * rows * el
    # matrix-core work of the factor kernels: 4H projections of C (the backward recomputes them)
    k_flops = 2 * rows * c * 4 * h
    peak = PEAK_BF16_TFLOPS if dtype == "bf16" else PEAK_F32_TFLOPS
    kern = lambda ms_, b_: {"ms": round(ms_, 4), "achieved_gbps": round(b_ / (ms_ * 1e-3) / 1e9, 1),  # noqa: E731
                            "frac": round(b_ / (ms_ * 1e-3) / 1e9 / 8000.0, 4),
                            "mfma_tflops": round(k_flops / (ms_ * 1e-3) / 1e12, 1),
                            "mfma_frac": round(k_flops / (ms_ * 1e-3) / 1e12 / peak, 4)}  # fmt: skip
    return {
        "workload": f"triangle_multiplication outgoing fwd+bwd, N={n}, C=H={c}, {dtype}, mask, biases",
        "ms_fwd_bwd": round(ms, 4),
        "ms_fwd": round(ms_fwd, 4),
        "tflops_fwd_bwd": round(flops / ms / 1e9, 2),
        "factor_kernel_fwd": kern(k_fwd, fwd_bytes),
        "factor_kernel_bwd": kern(k_bwd, bwd_bytes),
        "roofline_bound": "hbm" if dtype == "bf16" else "mfma (float32)",
    }


def layer_norm_stage(device, rows=512 * 512, width=128):
    """layer_norm fwd+bwd over 262144 x 128 bf16 rows (the pair LayerNorm at N=512) with float32 affine;
    HBM rate of the forward (x read, y written) and backward (x, dy read, dx written) against 8 TB/s."""

    import torch

    from oops_amd import layer_norm

    g = torch.Generator().manual_seed(14)
    x = torch.randn(rows, width, generator=g).to(torch.bfloat16).to(device).requires_grad_(True)
    w = torch.randn(width, generator=g).to(device).requires_grad_(True)
    b = torch.randn(width, generator=g).to(device).requires_grad_(True)
    dy = torch.randn(rows, width, generator=g).to(torch.bfloat16).to(device)
    with torch.no_grad():
        ms_fwd = _median_ms(lambda: layer_norm(x, width, w, b), iters=20, warmup=3)
    y = layer_norm(x, width, w, b)
    ms_bwd = _median_ms(lambda: torch.autograd.grad(y, [x, w, b], dy, retain_graph=True), iters=20, warmup=3)
    nbytes = rows * width * 2

    # the row kernels alone through the C ABI (the operator's times above add the custom-op host path and,
    # in the backward, the two float32 sums of the affine partials)
    import ctypes
    import importlib

    from oops_amd import _lib

    ln = importlib.import_module("oops_amd.normalization.layer_norm")
    lib = _lib.load()
    with torch.no_grad():
        xd = x.detach()
        yk, mean, rstd = (torch.empty_like(xd), torch.empty(rows, device=device), torch.empty(rows, device=device))
        dx = torch.empty_like(xd)
        geo = ln._geometry(xd.dtype, rows, width, width, 1e-5)
        parts = torch.empty(2, lib.oops_layer_norm_rows_parts(ctypes.byref(geo)), width, device=device)
        stream = torch.cuda.current_stream().cuda_stream
        k_fwd = _median_ms(lambda: lib.oops_layer_norm_rows_forward(
            ctypes.byref(geo), xd.data_ptr(), w.data_ptr(), b.data_ptr(), yk.data_ptr(), mean.data_ptr(),
            rstd.data_ptr(), stream), iters=20, warmup=3)  # fmt: skip
        k_bwd = _median_ms(lambda: lib.oops_layer_norm_rows_backward(
            ctypes.byref(geo), xd.data_ptr(), w.data_ptr(), mean.data_ptr(), rstd.data_ptr(), dy.data_ptr(),
            dx.data_ptr(), parts[0].data_ptr(), parts[1].data_ptr(), stream), iters=20, warmup=3)  # fmt: skip
    kern = lambda ms_, b_: {"ms": round(ms_, 4), "achieved_gbps": round(b_ / (ms_ * 1e-3) / 1e9, 1),  # noqa: E731
                            "frac": round(b_ / (ms_ * 1e-3) / 1e9 / 8000.0, 4)}  # fmt: skip
    return {
        "workload": f"layer_norm {rows} x {width} bf16, float32 affine",
        "ms_fwd": round(ms_fwd, 4),
        "fwd_gbps": round(2 * nbytes / (ms_fwd * 1e-3) / 1e9, 1),
        "ms_bwd": round(ms_bwd, 4),
        "bwd_gbps": round(3 * nbytes / (ms_bwd * 1e-3) / 1e9, 1),
        # forward kernel: x read, y written (+ 2 float32 statistics per row); backward: x, dy read, dx written
        "forward_kernel": kern(k_fwd, 2 * nbytes + 8 * rows),
        "backward_kernel": kern(k_bwd, 3 * nbytes + 8 * rows),
        "peak_gbps": 8000.0,
    }


def gate_stage(device):
    """The gated output stage (the row after attention) at config 4's MSA shape.

    rows = S x N = 512 x 384 tokens, H = 8, D = 32 (gate width 256), single
    C = 256, output width 256, bf16.  Reports the fused gate-projection kernel
    (logits GEMM + sigmoid + product, HIP events on its launch stream) against
    HBM, the backward elementwise kernel likewise, and the whole
    gate_attention_output fwd+bwd (which adds the output projection and the
    weight/single gradients as library GEMMs).
    """

    import torch

    from oops_amd import gate_attention_output
    from oops_amd.attention import gate as gate_mod

    s_, n, h, d, c, o = 512, 384, 8, 32, 256, 256
    g = torch.Generator().manual_seed(3)
    att = torch.randn(s_, n, h, d, generator=g).to(torch.bfloat16).to(device).permute(0, 2, 1, 3)  # (S, H, N, D)
    single = torch.randn(s_, n, c, generator=g).to(torch.bfloat16).to(device)
    w = (torch.randn(h * d, c, generator=g) / c**0.5).to(torch.bfloat16).to(device)
    wo = (torch.randn(o, h * d, generator=g) / (h * d) ** 0.5).to(torch.bfloat16).to(device)
    dy = torch.randn(s_, n, o, generator=g).to(torch.bfloat16).to(device)
    rows, width = s_ * n, h * d
    att5 = att.transpose(-3, -2).unsqueeze(0)
    single_rows = single.reshape(rows, c)
    stream = torch.cuda.current_stream()
    fwd = lambda: gate_mod.gate_forward(att5, single_rows, w, True)
    gated, logits = fwd()
    # the projection kernel alone through the C ABI on the operator's own operands (the Python wrapper's
    # host work per call would otherwise be part of the time)
    import ctypes

    from oops_amd import _lib

    lib = _lib.load()
    geo = gate_mod._gate_geometry(att5, single_rows, w)
    ptrs = [t.data_ptr() for t in (single_rows, w, att5, gated, logits)]

    def proj():
        rc = lib.oops_gate_projection_forward(ctypes.byref(geo), *ptrs, stream.cuda_stream)
        assert rc == 0, lib.oops_last_error()

    fwd_ms = time_events_batched(proj, 10, 3, stream)
    grad = torch.randn(rows, width, generator=g).to(torch.bfloat16).to(device)
    bwd = lambda: gate_mod.gate_backward(grad, att5, logits, True, True)
    bwd_ms = time_events_batched(bwd, 10, 3, stream)
    fwd_bytes = 2 * (rows * c + width * c + 3 * rows * width)  # single, W, attention read; gated, logits written
    bwd_bytes = 2 * 5 * rows * width  # logits, grad, attention read; two gradients written
    leaves = [t.requires_grad_(True) for t in (att, single, w, wo)]

    def step():
        out = gate_attention_output(*leaves)
        torch.autograd.grad(out, leaves, dy)

    step_ms = _median_ms(step)
    return {
        "workload": "gate_attention_output fwd+bwd, rows 512x384, H=8, D=32, C=256, O=256, bf16",
        "ms_fwd_bwd": round(step_ms, 4),
        "projection_kernel": {
            "ms": round(fwd_ms, 4),
            "bound": "hbm",
            "achieved_gbps": round(fwd_bytes / fwd_ms / 1e6, 1),
            "peak_gbps": 8000.0,
            "frac": round(fwd_bytes / fwd_ms / 1e6 / 8000.0, 4),
            "tflops": round(2 * rows * width * c / fwd_ms / 1e9, 1),
        },
        "backward_kernel": {
            "ms": round(bwd_ms, 4),
            "bound": "hbm",
            "achieved_gbps": round(bwd_bytes / bwd_ms / 1e6, 1),
            "frac": round(bwd_bytes / bwd_ms / 1e6 / 8000.0, 4),
        },
    }


def cpu_baseline(budget_s=15.0):
    """The numpy oracle (float32) on a bounded sample of rows of the same workload."""

    import numpy as np

    from oracle import attention as ora

    try:
        from threadpoolctl import threadpool_info

        threads = max((i.get("num_threads", 1) for i in threadpool_info()), default=1)
    except Exception:  # pragma: no cover
        threads = 1
    rng = np.random.default_rng(2)
    bias = rng.standard_normal((1, 1, H, N, N), dtype=np.float32)
    rows_done, elapsed, chunk = 0, 0.0, 4
    while elapsed < budget_s and rows_done < N:
        q, k, v, do = (rng.standard_normal((1, chunk, N, H, C), dtype=np.float32) for _ in range(4))
        t0 = time.perf_counter()
        ora.triangle_attention_forward(q, k, v, None, bias, dtype=np.float32)
        ora.triangle_attention_backward(q, k, v, do, None, bias, dtype=np.float32)
        elapsed += time.perf_counter() - t0
        rows_done += chunk
    flops = 14 * H * C * N * N * rows_done
    return {
        "value": flops / elapsed / 1e12,
        "unit": "TFLOP/s",
        "cores": int(threads),
        "kind": "port",
        "sample": f"numpy float32 oracle fwd+bwd on {rows_done} of {N} rows (N={N}, H={H}, c={C}, shared bias), "
        f"{elapsed:.1f} s; host os.cpu_count()={os.cpu_count()}",
        "ms_per_call_extrapolated": elapsed / rows_done * N * 1e3,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--no-extra", action="store_true", help="skip the configs 2/4/5 timings")
    ap.add_argument(
        "--copy-calibration",
        action="store_true",
        help="only copy a 256 MiB device buffer 3 times (scales rocprofv3 FETCH_SIZE/WRITE_SIZE readings)",
    )
    ap.add_argument(
        "--only",
        choices=("nested_msa", "layer_norm", "trimul_f32", "c2", "c4", "c5"),
        help="only measure one of the rows beside attention (3 repetitions) and print its JSON",
    )
    ap.add_argument(
        "--trimul-only",
        action="store_true",
        help="only measure triangle_multiplication (N=512, C=H=128, 3 repetitions) and print its JSON",
    )
    ap.add_argument(
        "--gate-only",
        action="store_true",
        help="only measure the gated output stage at config 4's MSA shape (3 repetitions) and print its JSON",
    )
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(
            "bench.py measures one GPU only: this build has no multi-GPU path "
            "(rows shard independently across GPUs; one GPU's share is what this measures). Run with --gpus 1.",
            file=sys.stderr,
        )
        sys.exit(2)

    import torch

    if args.copy_calibration:
        x = torch.empty(COPY_CAL_BYTES // 4, device="cuda:0")
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()
        return

    from oops_amd import _lib

    _lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.only:
        fn = {"nested_msa": nested_msa, "layer_norm": layer_norm_stage,
              "trimul_f32": lambda d: trimul_stage(d, dtype="f32"),
              **{c: (lambda d, c=c: other_configs(d, (c,))) for c in ("c2", "c4", "c5")}}[args.only]
        for _ in range(3):
            res = fn(dev)
        print(json.dumps(res))
        return
    if args.trimul_only:
        for _ in range(3):
            res = trimul_stage(dev)
        print(json.dumps(res))
        return
    if args.gate_only:
        for _ in range(3):
            gate = gate_stage(dev)
        print(json.dumps(gate))
        return
    q, k, v, bias, dout = make_inputs(dev)
    torch.cuda.synchronize()
    _log("bench: warmup")
    for _ in range(args.warmup):
        step(q, k, v, bias, dout)
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(args.steps):
        step(q, k, v, bias, dout)
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(end) / args.steps
    peak_mem = torch.cuda.max_memory_allocated()
    _log(f"bench: {ms:.3f} ms/step (wall {wall / args.steps * 1e3:.3f} ms)")
    # the survey's timing rule beside the driver's mean: median of 50 steps, each between its own event
    # pair, after 10 warm-ups
    ms_med50 = time_events(lambda: step(q, k, v, bias, dout), 50, 10, stream)
    _log(f"bench: median of 50 steps {ms_med50:.3f} ms")

    kt = kernel_times(q, k, v, bias, dout)
    _log("bench: kernel ms " + json.dumps({k_: round(v_, 4) for k_, v_ in kt.items()}))
    dominant = max(kt, key=kt.get)
    unit_flops = 2 * H * C * N**3
    ach = KERNEL_GEMMS[dominant] * unit_flops / (kt[dominant] * 1e-3) / 1e12
    value = flops_step() / (ms * 1e-3) / 1e12
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "ms_per_step_median50": round(ms_med50, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded randn, BASELINE config 3)",
        "config": {
            "workload": "triangle attention ending node fwd+bwd (config 3)",
            "N": N,
            "heads": H,
            "head_size": C,
            "bias": "shared [1,1,4,768,768] bf16",
            "mask": None,
            "parallelism": "single GPU",
        },
        # algorithmic FLOP/s of the whole step over the dense bf16 peak
        "flops_frac_of_peak": round(value / PEAK_BF16_TFLOPS, 4),
        # MFMA busy cycles over all SIMD cycles, per kernel, from the committed rocprofv3 counters
        # (profiles/triangle_attention_c3_bf16_mfma.txt); includes the identity-MFMA bias adds
        "mfma_util_pct": measured_mfma() or None,
        "bias_traffic": bias_traffic(kt),
        "peak_mem_bytes": int(peak_mem),
        "kernel_ms": {k_: round(v_, 4) for k_, v_ in kt.items()},
        "roofline": {
            "kernel": dominant,
            "bound": "mfma",
            "achieved": round(ach, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(ach / PEAK_BF16_TFLOPS, 4),
            "traffic": measured_traffic(dominant),
        },
    }
    if not args.no_extra:
        _log("bench: configs 2, 4, 5")
        line["other_configs"] = other_configs(dev)
        _log("bench: " + json.dumps(line["other_configs"]))
        _log("bench: gated output stage")
        line["next_rows"] = {"gate_c4_shape": gate_stage(dev), "nested_msa": nested_msa(dev),
                             "trimul_n512": trimul_stage(dev), "trimul_n512_f32": trimul_stage(dev, dtype="f32"),
                             "layer_norm": layer_norm_stage(dev)}
        _log("bench: " + json.dumps(line["next_rows"]))
    if not args.no_cpu:
        _log("bench: accuracy against the oracle")
        line["accuracy"] = accuracy(q, k, v, bias, dout)
        _log("bench: cpu baseline")
        line["cpu_baseline"] = cpu_baseline(args.cpu_budget)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
