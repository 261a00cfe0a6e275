#!/usr/bin/env python
"""Benchmark of the GOAP quantized-linear path on one MI355X.

Metric: QuantLinear M=1 HBM GB/s (% of 8 TB/s peak) and
M=2048 TFLOPS (% of the 2.5 PFLOP/s dense bf16 MFMA peak).

Workload (`value`): decode at M=1 through the seven linears of a
Llama-3-8B-shaped decoder layer (q 4096x4096, k/v 1024x4096, o 4096x4096,
gate/up 14336x4096, down 4096x14336), 4-bit NF4 + double quant, group 128,
0.1 % outliers (the 4-bit M=1 decode target). One step is
one layer forward: the seven QuantLinear forwards in four launches, q/k/v and
gate/up each one grouped launch over layers that share their input
(QuantLinear.forward_group), o and down one launch each (--ungrouped: seven
launches). Ten copies of the layer (1.2 GB) are rotated so every step streams
its weights from HBM and not from the 256 MB MALL: one captured HIP graph
holds ten consecutive steps, one per copy, as a ten-layer model's decode
graph would. Each launch reads the activation the launch before it wrote (of
the width it needs; the first launch of a replay reads a resident input), as
every linear of a decoder layer does.

Alongside it (extra keys of the same JSON line):
  * "roofline"       - the decode kernel: algorithmic bytes of a step's launches /
                       the sum of their average durations (HIP events around
                       graph replays of each launch over the copies), vs 8 TB/s;
  * "decode_drop_in" - the same step as a caller of the reference API runs it:
                       one QuantLinear.forward per linear, 7 launches
                       ("decode_grouped" with --ungrouped);
  * "cfg1"           - BASELINE config 1: the 4096x4096 linear by itself at
                       M = 1 and 16, each line with the reference CPU fallback
                       forward of the same layer timed beside it;
  * "cfg2"           - BASELINE config 2: the 11008x4096 2-bit companded
                       (Lloyd-Max) linear by itself at M = 1, 4 and 8, with the
                       reference CPU fallback forward beside each line;
  * "decode_cfg5"    - the same decode step on BASELINE config 5's 70B layer
                       (its 8/4/2-bit mix), 3 rotating copies (1.4 GB);
  * "prefill"        - BASELINE config 4: gate/up/down at M=2048, 8-bit NF8 + DQ
                       and 6-bit RVQ, 2*M*N*K flops / GPU time vs 2.5 PFLOP/s,
                       through QuantLinear.forward (the fused dequant-into-LDS
                       MFMA kernel), with dequantize + hipBLASLt GEMM beside it
                       as "library_reference"; "short_prompt": M=256 through
                       config 3's seven 4-bit linears (the fused kernel
                       splitting K where few tiles) beside the same library
                       reference;
  * "quantize"       - BASELINE config 5's GPU GOAP quantize (28672x8192) through
                       the public API, wall time, with the oracle CPU codec timed
                       on the same full weight;
  * "cpu_baseline"   - the reference CPU fallback forward (bf16 dequant + F.linear,
                       modules.py:752-804, 924-940), restated in oracle/, timed
                       on this host's cores for one layer forward at M=1.
Synthetic seeded weights/activations (tests/golden/recipes.py).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def layer_bytes(ql, M: int) -> int:
    """Algorithmic bytes of one decode launch: every byte the launch must move
    once, i.e. packed codes + metadata + outlier tables + codebook + x + y
    (+ bias)."""
    N, K = ql.out_features, ql.in_features
    b = ql.packed.numel()
    if ql.double_quant:
        b += ql.dq_scale_codes.numel() + ql.dq_gmin_codes.numel()
        b += (ql.dq_scale_meta.numel() + ql.dq_gmin_meta.numel()) * 2
    else:
        b += (ql.scale.numel() + ql.gmin.numel()) * 2
    if ql.bits == 6:
        b += ql.stage2_packed.numel() + (ql.stage2_scale.numel() + ql.stage2_gmin.numel()) * 2
    b += ql.outlier_row.numel() * (4 + 4 + 2)
    if ql.codebook is not None:
        b += ql.codebook.numel() * 4
    b += M * K * 2 + M * N * 2
    if ql.bias is not None:
        b += N * 2
    return int(b)


def clone_layer(ql):
    """A second QuantLinear over fresh copies of the same buffers and derived
    outlier tables."""
    import copy
    c = copy.copy(ql)
    c._buffers = {k: (v.clone() if v is not None else None) for k, v in ql._buffers.items()}
    for name in ql._DERIVED:
        c.__dict__[name] = ql.__dict__[name].clone()
    c._rebuild_cache()
    return c


def build_decode_layer(linears, opts_of, sigma=0.02, seed0=1000):
    """Quantized QuantLinears of one decoder layer: (name, out, in) shapes,
    per-linear quantize options, seeded N(0, sigma) weights with outliers."""
    import recipes
    import tensorshrink_amd as ts
    layer = []
    for i, (name, n, k) in enumerate(linears):
        w = recipes.gaussian_weight(n, k, seed0 + i, sigma=sigma)
        t0 = time.time()
        qt = ts.quantize_tensor(w, **opts_of(name))
        ql = ts.QuantLinear(qt)
        log(f"  quantized {name} {n}x{k} in {time.time() - t0:.2f}s")
        layer.append((name, ql))
        del w
    return layer


# the 70B layer's adaptive mix (attention 8-bit, MLP 4-bit,
# down 2-bit companded).
CFG5_OPTS = {
    **{n: dict(bits=8, group_size=128, outlier_frac=0.001, double_quant=True, nf_quant=True)
       for n in ("q", "k", "v", "o")},
    **{n: dict(bits=4, group_size=128, outlier_frac=0.001, double_quant=True, nf_quant=True)
       for n in ("gate", "up")},
    "down": dict(bits=2, group_size=64, outlier_frac=0.001, double_quant=True, companded=True),
}

# Launches of one decode step: (name, positions in LLAMA3_8B_LINEARS).
GROUPED_UNITS = [("qkv", (0, 1, 2)), ("o", (3,)), ("gate_up", (4, 5)), ("down", (6,))]
SINGLE_UNITS = [(n, (i,)) for i, n in enumerate(("q", "k", "v", "o", "gate", "up", "down"))]


def run_unit(layer, idx, xs, live=None):
    """The forwards of one launch unit (a list of outputs). With `live`, the
    input is the latest output of the input's width (the activation the
    previous launch just wrote, as in a model's decode step, where every
    linear reads what the kernel before it produced), and the unit's outputs
    become the latest of their widths."""
    import tensorshrink_amd as ts
    qs = [layer[i][1] for i in idx]
    src = live if live is not None else xs
    x = src[qs[0].in_features]
    ys = [qs[0](x)] if len(qs) == 1 else ts.QuantLinear.forward_group(qs, x)
    if live is not None:
        seen = set()
        for y in ys:
            if y.shape[-1] not in seen:
                live[y.shape[-1]] = y
                seen.add(y.shape[-1])
    return ys


def build_copies(linears, opts_of, n_copies, sigma=0.02, seed0=1000):
    """A decoder layer and n_copies - 1 clones of it (rotated through so no
    step finds its weights in the 256 MB MALL)."""
    torch.cuda.synchronize()
    base = build_decode_layer(linears, opts_of, sigma, seed0)
    return [base] + [[(n, clone_layer(q)) for n, q in base] for _ in range(n_copies - 1)]


def bench_decode(args, linears, opts_of, n_copies, steps, warmup, kernel_reps, sigma=0.02, seed0=1000,
                 copies=None, units=None):
    import recipes
    if copies is None:
        copies = build_copies(linears, opts_of, n_copies, sigma, seed0)
    base = copies[0]
    widths = sorted({k for _, _, k in linears})
    xs = {k: recipes.activations(1, k).cuda() for k in widths}
    step_bytes = sum(layer_bytes(q, 1) for _, q in base)
    if units is None:
        units = SINGLE_UNITS if args.ungrouped else GROUPED_UNITS
    stream = torch.cuda.Stream()
    C = len(copies)
    full, rem = divmod(steps, C)
    outs = []
    with torch.cuda.stream(stream):
        for layer in copies:  # warm every kernel instantiation outside capture
            for _, idx in units:
                run_unit(layer, idx, xs)
        torch.cuda.synchronize()

        def capture(n):  # one graph: n consecutive steps, step i on copy i, chained
            g = torch.cuda.CUDAGraph()
            live = dict(xs)
            with torch.cuda.graph(g, stream=stream):
                for layer in copies[:n]:
                    outs.append([run_unit(layer, idx, xs, live) for _, idx in units])
            return g
        g_all = capture(C)
        g_rem = capture(rem) if rem else None
        torch.cuda.synchronize()
        for _ in range(max(1, -(-warmup // C))):
            g_all.replay()
        torch.cuda.synchronize()
        # timed region: exactly K steps, as K // C replays of the C-step graph
        # and one of a K % C-step graph; HIP events around each replay on the
        # replay stream
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True), C)
               for _ in range(full)]
        if rem:
            evs.append((torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True), rem))
        t0 = time.perf_counter()
        for i, (e0, e1, n) in enumerate(evs):
            e0.record(stream)
            (g_all if n == C else g_rem).replay()
            e1.record(stream)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    step_gpu_ms = sum(a.elapsed_time(b) for a, b, _ in evs) / steps
    kern = unit_kernel_time(copies, xs, stream, units, reps=kernel_reps)
    return dict(ms_per_step=ms_per_step, value=value, step_bytes=step_bytes, kern=kern,
                base=base, xs=xs, step_gpu_us=step_gpu_ms * 1e3, units=units, copies=copies)


def bench_single(copies, idx: int, M: int, reps: int):
    """One linear of the layer by itself (BASELINE config 1 is the layer's
    4096x4096 q shape): a graph holding its forward on every copy back to
    back at M tokens, replayed `reps` times between HIP events on the launch
    stream. Per-launch average (dispatch gap included)."""
    import recipes
    q0 = copies[0][idx][1]
    x = recipes.activations(M, q0.in_features, seed=M).cuda()
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for layer in copies:
            layer[idx][1](x)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for layer in copies:
                layer[idx][1](x)
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (reps * len(copies))
    nb = layer_bytes(q0, M)
    return {"M": M, "bytes": nb, "us": round(us, 2), "GBps": round(nb / (us * 1e-6) / 1e9, 1),
            "frac_of_hbm_peak": round(nb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def bench_cfg2(args, n_copies=24):
    """one 11008x4096 QuantLinear, 2-bit companded
    (Lloyd-Max codebook fitted per tensor), group 64, outlier_frac 0.001,
    Student-t(5) x 0.02 weights (the test suite's seeds), at M = 1, 4 and 8.
    24 rotating copies (about 310 MB) so that a replay does not find its
    weights in the 256 MB MALL."""
    import recipes
    import tensorshrink_amd as ts
    torch.manual_seed(2024)  # the Lloyd-Max fit samples from the global RNG
    w = recipes.student_t_weight(11008, 4096, 2000)
    base = ts.QuantLinear(ts.quantize_tensor(w, bits=2, group_size=64, outlier_frac=0.001, companded=True))
    del w
    copies = [[("cfg2", base)]] + [[("cfg2", clone_layer(base))] for _ in range(n_copies - 1)]
    lines = [bench_single(copies, 0, M, args.kernel_reps * 3) for M in (1, 4, 8)]
    if not args.no_cpu:
        for line in lines:
            line["cpu_baseline"] = cpu_forward_baseline(base, line["M"], min(args.cpu_budget, 8.0))
    del copies
    torch.cuda.empty_cache()
    return {"workload": "BASELINE config 2: single QuantLinear 11008x4096, 2-bit companded (Lloyd-Max), group 64, "
                        "outlier_frac 0.001, Student-t(5) weights; one launch per forward, 24 rotating copies",
            "lines": lines}


def cpu_forward_baseline(ql, M: int, budget_s: float):
    """The reference CPU fallback forward (oracle restatement: bf16 dequant
    + F.linear, modules.py:752-804, 924-940) of one linear at M tokens,
    timed on this host's cores (median of up to 10 runs within budget_s)."""
    import recipes
    from oracle import codec_ref as O
    torch.set_num_threads(os.cpu_count() or 1)
    qt = ql.to_quantized_tensor()
    q = dict(packed=qt.packed, scale=qt.scale, gmin=qt.gmin, outlier_idx=qt.outlier_idx,
             outlier_val=qt.outlier_val, dq_scale_codes=qt.dq_scale_codes, dq_scale_meta=qt.dq_scale_meta,
             dq_gmin_codes=qt.dq_gmin_codes, dq_gmin_meta=qt.dq_gmin_meta, codebook=qt.codebook,
             _meta=dict(bits=qt.bits, group_size=qt.group_size, rows=qt.rows, cols=qt.cols,
                        padded_cols=qt.padded_cols, n_groups=qt.n_groups, orig_dtype=qt.orig_dtype))
    bufs = dict(outlier_row=ql.outlier_row.cpu().numpy(), outlier_col=ql.outlier_col.cpu().numpy(),
                outlier_delta=ql.outlier_delta.cpu().numpy())
    x = recipes.activations(M, ql.in_features, seed=M)
    O.quantlinear_forward_cpu(q, bufs, x)  # warmup
    times, t_start = [], time.perf_counter()
    while len(times) < 2 or (time.perf_counter() - t_start < budget_s and len(times) < 10):
        t0 = time.perf_counter()
        O.quantlinear_forward_cpu(q, bufs, x)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    nb = layer_bytes(ql, M)
    return {"value": round(nb / med / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(), "kind": "port",
            "us": round(med * 1e6, 1), "sample": f"{len(times)} CPU forwards at M={M} (median)"}


def unit_kernel_time(copies, xs, stream, units, reps: int):
    """Average decode launch duration per launch unit in isolation: one graph
    per unit holding that unit's launch on every copy (back to back, the
    weights rotating so none comes from the MALL, x a resident tensor that
    the weight stream evicts from the caches), replayed `reps` times between
    two HIP events on the launch stream. The per-launch average includes the
    dispatch gap between consecutive kernels of a graph."""
    out = {}
    with torch.cuda.stream(stream):
        graphs = []
        for name, idx in units:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for layer in copies:
                    run_unit(layer, idx, xs)
            graphs.append((name, idx, g))
        for _, _, g in graphs:
            g.replay()
        torch.cuda.synchronize()
        evs = []
        for name, idx, g in graphs:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(reps):
                g.replay()
            e1.record(stream)
            evs.append((name, idx, e0, e1))
        torch.cuda.synchronize()
    for name, idx, e0, e1 in evs:
        us = e0.elapsed_time(e1) * 1e3 / (reps * len(copies))
        qs = [copies[0][i][1] for i in idx]
        nb = sum(layer_bytes(q, 1) for q in qs)
        out[name] = {"shapes": [[q.out_features, q.in_features] for q in qs], "bytes": nb, "us": round(us, 2),
                     "GBps": round(nb / (us * 1e-6) / 1e9, 1)}
    return out


def load_traffic(units):
    """HBM bytes per launch from the committed PMC summary (FETCH_SIZE and
    WRITE_SIZE passes of rocprofv3 over this bench, each scaled by the same
    counter's reading for a plain copy of known size), or None when the
    summary does not cover these launch units."""
    path = os.path.join(ROOT, "profiles", "decode_traffic.json")
    if not os.path.exists(path):
        return None
    try:
        per = json.load(open(path))["per_launch_bytes"]
        pu = {u: int(per[u]) for u, _ in units}
        return {"bytes_per_step": int(sum(pu.values())), "per_launch_bytes": pu,
                "source": "profiles/decode_traffic.json"}
    except (OSError, KeyError, ValueError):
        return None


def decode_counter_launches(n=50):
    """Eager M = 1 forwards for SQ-counter runs (no graphs, no timing): the
    config-2 layer (2-bit Lloyd-Max, group 64), a 4096 x 4096 and a 14336 x
    4096 NF4 + double-quant layer, n launches each."""
    import recipes
    import tensorshrink_amd as ts
    nf4 = dict(bits=4, group_size=128, outlier_frac=0.001, double_quant=True, nf_quant=True)
    lm2 = dict(bits=2, group_size=64, outlier_frac=0.001, companded=True)
    for name, fmt, rows, cols in (("cfg2", lm2, 11008, 4096), ("nf4_4096", nf4, 4096, 4096),
                                  ("nf4_14336", nf4, 14336, 4096)):
        torch.manual_seed(1)
        ql = ts.QuantLinear(ts.quantize_tensor(recipes.gaussian_weight(rows, cols, 3), **fmt))
        x = recipes.activations(1, cols, seed=1).cuda()
        for _ in range(n):
            ql(x)
        torch.cuda.synchronize()
        log(f"decode counters: {name} x {n}")
        del ql


def copy_calibration():
    """A plain device copy of known size, for scaling FETCH_SIZE/WRITE_SIZE."""
    n = 512 * 1024 * 1024
    src = torch.empty(n, dtype=torch.uint8, device="cuda").random_(0, 255)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n, "launches": 5}), flush=True)


def _forward_gemm(q, x):
    """ts_qlinear_forward with a workspace: dequantize into it + one hipBLASLt
    GEMM (the library reference for the fused kernel)."""
    import ctypes
    from tensorshrink_amd import _lib as L
    lib = L.load()
    y = torch.empty(x.shape[0], q.out_features, dtype=x.dtype, device=x.device)
    n = lib.ts_forward_workspace_bytes(ctypes.byref(q._layer), x.shape[0])
    ws = _WS.get(n)
    if ws is None:
        _WS.clear()
        ws = _WS[n] = torch.empty(n, dtype=torch.uint8, device=x.device)
    dt = L.dtype_code(x.dtype)
    L.check(lib.ts_qlinear_forward(ctypes.byref(q._layer), x.data_ptr(), x.shape[0], q.in_features, dt,
                                   y.data_ptr(), q.out_features, dt, None, ws.data_ptr(), n, L.stream_ptr()),
            "dequant + gemm")
    return y


_WS: dict = {}


def _timed_linears(lins, xs, M, fwd, steps):
    """Per-linear GPU time (HIP events, one round of warmup absorbed) of
    fwd(q, x) over `steps` rounds of the linears; TFLOPS over all of them."""
    flops = {name: 2.0 * M * q.out_features * q.in_features for name, q in lins}
    for _, q in lins:
        fwd(q, xs[q.in_features])
    torch.cuda.synchronize()
    times = {name: [] for name, _ in lins}
    evs = []
    for s in range(steps):
        for name, q in lins:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fwd(q, xs[q.in_features])
            e1.record()
            evs.append((name, e0, e1))
    torch.cuda.synchronize()
    for name, e0, e1 in evs[len(lins):]:  # the first round absorbs the empty-queue start
        times[name].append(e0.elapsed_time(e1))
    tot_f = sum(flops[n] * len(times[n]) for n in times)
    tot_ms = sum(sum(times[n]) for n in times)
    tflops = tot_f / (tot_ms * 1e-3) / 1e12
    return {"tflops": round(tflops, 1), "frac": round(tflops / BF16_PEAK_TFLOPS, 4),
            "per_linear_us": {n: round(sum(t) / len(t) * 1e3, 1) for n, t in times.items()},
            "layer_us": round(sum(sum(t) / len(t) for t in times.values()) * 1e3, 1)}


def bench_prefill(args):
    import recipes
    import tensorshrink_amd as ts
    res = {}
    M = 2048
    for bits in (8, 6):
        opts = dict(bits=bits, group_size=128, outlier_frac=0.001, double_quant=True, nf_quant=True)
        lins = []
        for i, (name, n, k) in enumerate(recipes.LLAMA3_8B_LINEARS[4:]):
            w = recipes.gaussian_weight(n, k, recipes.layer_seed(4 + i))
            lins.append((name, ts.QuantLinear(ts.quantize_tensor(w, **opts))))
            del w
        xs = {4096: recipes.activations(M, 4096).cuda(), 14336: recipes.activations(M, 14336).cuda()}

        def timed(fwd):
            r = _timed_linears(lins, xs, M, fwd, args.prefill_steps)
            r.pop("layer_us")
            return r

        r = timed(lambda q, x: q(x))
        r["path"] = ("QuantLinear.forward: the fused dequant-into-LDS MFMA kernel (ts::prefill_kernel, "
                     "256x256 tiles, 8 waves; the down projection's K split in two, fp32 partials + one "
                     "reduction pass)")
        lib_ref = timed(_forward_gemm)
        lib_ref["path"] = "library reference: dequantize into a workspace + one hipBLASLt GEMM"
        r["library_reference"] = lib_ref
        res[f"{bits}bit"] = r
        _WS.clear()
        del lins, xs
        torch.cuda.empty_cache()
    return res


def bench_prefill_short(args, M=256):
    """A short prompt through the whole config-3 layer (q, k, v, o, gate, up,
    down; 4-bit NF4 + double quant, group 128): QuantLinear.forward, whose
    fused kernel splits K across workgroups where its tiles would leave CUs
    idle, against dequantize + hipBLASLt."""
    import recipes
    import tensorshrink_amd as ts
    opts = dict(bits=4, group_size=128, outlier_frac=0.001, double_quant=True, nf_quant=True)
    lins = []
    for i, (name, n, k) in enumerate(recipes.LLAMA3_8B_LINEARS):
        w = recipes.gaussian_weight(n, k, recipes.layer_seed(i))
        lins.append((name, ts.QuantLinear(ts.quantize_tensor(w, **opts))))
        del w
    xs = {4096: recipes.activations(M, 4096).cuda(), 14336: recipes.activations(M, 14336).cuda()}
    r = _timed_linears(lins, xs, M, lambda q, x: q(x), args.prefill_steps)
    r["path"] = "QuantLinear.forward per linear (fused prefill kernel, K split where few tiles)"
    lib_ref = _timed_linears(lins, xs, M, _forward_gemm, args.prefill_steps)
    lib_ref["path"] = "library reference: dequantize into a workspace + one hipBLASLt GEMM"
    r["library_reference"] = lib_ref
    r["workload"] = (f"M={M} through the config-3 Llama-3-8B layer's 7 linears, 4-bit NF4 + double quant, "
                     "group 128, outlier_frac 0.001")
    _WS.clear()
    del lins, xs
    torch.cuda.empty_cache()
    return r


def bench_quantize(args):
    """BASELINE config 5's GPU GOAP quantize: the 28672x8192 fp16 N(0, 0.015)
    weight with outliers, 4-bit uniform, group 128, outlier_frac 0.001 (the
    gpu_quantize.py flavour), through the public API (quantize_tensor returns
    host numpy arrays, as the reference's does). Wall time per call with the
    weight resident on the GPU; algorithmic bytes = read N*K*2 + write packed
    + scale/gmin + outliers (i32 index + fp16 value). The reference CPU codec,
    restated in oracle/ (libstdc++ top-k + numpy), is timed once on the same
    full weight on this host's cores."""
    import numpy as np
    import recipes
    import tensorshrink_amd as ts
    from oracle import codec_ref as O
    N, K, gs, frac = 28672, 8192, 128, 0.001
    w = recipes.gaussian_weight(N, K, 5005, sigma=0.015).cuda()
    opts = dict(bits=4, group_size=gs, outlier_frac=frac)
    ts.quantize_tensor(w, **opts)
    torch.cuda.synchronize()
    times = []
    for _ in range(args.quantize_reps):
        t0 = time.perf_counter()
        qt = ts.quantize_tensor(w, **opts)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    k = max(1, int(N * K * frac))
    nbytes = N * K * 2 + qt.packed.nbytes + qt.scale.nbytes + qt.gmin.nbytes + k * (4 + 2)
    res = {"workload": "GOAP quantize 28672x8192 fp16 -> 4-bit uniform, group 128, outlier_frac 0.001 "
                       "(BASELINE config 5), host numpy result",
           "ms": round(med * 1e3, 2), "bytes": nbytes, "GBps": round(nbytes / med / 1e9, 2),
           "frac_of_hbm_peak": round(nbytes / med / 1e9 / HBM_PEAK_GBS, 5)}
    if not args.no_cpu:
        wc = w.cpu()
        torch.set_num_threads(os.cpu_count() or 1)
        t0 = time.perf_counter()
        O.quantize(wc, bits=4, group_size=gs, outlier_frac=frac)
        t = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": round(nbytes / t / 1e9, 4), "unit": "GB/s", "cores": torch.get_num_threads(),
                               "kind": "port", "ms": round(t * 1e3, 1),
                               "sample": f"oracle CPU quantize of the same full {N}x{K} weight (k = {k}), one call"}
        del wc
    del w
    torch.cuda.empty_cache()
    return res


def bench_quantize_module(args):
    """quantize_module over BASELINE config 5's layer (q/k/v/o, gate/up/down of
    the 70B shape, fp16 CPU weights as a model holds them before it moves to
    the GPU), NF4 + double quant (quantize_module's defaults), wall time with
    one and with four top-k replay workers (the layers' heap replays then run
    in parallel; results are identical)."""
    import recipes
    import tensorshrink_amd as ts
    lins = recipes.LLAMA3_70B_LINEARS
    ws = [recipes.gaussian_weight(n, k, 5200 + i, sigma=0.015) for i, (_, n, k) in enumerate(lins)]
    nbytes = sum(w.numel() * 2 for w in ws)

    def model():
        m = torch.nn.Module()
        for (name, n, k), w in zip(lins, ws):
            lin = torch.nn.Linear(k, n, bias=False, dtype=torch.float16)
            lin.weight.data = w
            m.add_module(name, lin)
        return m
    res = {"workload": "quantize_module over the config-5 layer's 7 linears (855 M fp16 weights on the host), "
                       "NF4 + double quant, group 128, outlier_frac 0.001", "bytes": nbytes}
    for workers in (1, 4):
        m = model()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ts.quantize_module(m, verbose=False, quantize_workers=workers, skip_name_patterns=())
        torch.cuda.synchronize()
        t = time.perf_counter() - t0
        res[f"workers_{workers}"] = {"s": round(t, 3), "GBps": round(nbytes / t / 1e9, 2)}
        del m
        torch.cuda.empty_cache()
    return res


def cpu_baseline(dec, budget_s: float):
    """Time the reference CPU fallback forward (oracle restatement) for one
    layer at M=1, on this host's cores, with the layer's own codes."""
    import numpy as np
    from oracle import codec_ref as O
    torch.set_num_threads(os.cpu_count() or 1)
    layer = dec["base"]
    qs = []
    for name, ql in layer:
        qt = ql.to_quantized_tensor()
        q = dict(packed=qt.packed, scale=qt.scale, gmin=qt.gmin, outlier_idx=qt.outlier_idx,
                 outlier_val=qt.outlier_val, dq_scale_codes=qt.dq_scale_codes, dq_scale_meta=qt.dq_scale_meta,
                 dq_gmin_codes=qt.dq_gmin_codes, dq_gmin_meta=qt.dq_gmin_meta, codebook=qt.codebook,
                 _meta=dict(bits=qt.bits, group_size=qt.group_size, rows=qt.rows, cols=qt.cols,
                            padded_cols=qt.padded_cols, n_groups=qt.n_groups, orig_dtype=qt.orig_dtype))
        bufs = dict(outlier_row=ql.outlier_row.cpu().numpy(), outlier_col=ql.outlier_col.cpu().numpy(),
                    outlier_delta=ql.outlier_delta.cpu().numpy())
        qs.append((q, bufs, dec["xs"][ql.in_features].cpu()))
    def one():
        for q, b, x in qs:
            O.quantlinear_forward_cpu(q, b, x)
    one()  # warmup
    times = []
    t_start = time.perf_counter()
    while len(times) < 2 or (time.perf_counter() - t_start < budget_s and len(times) < 10):
        t0 = time.perf_counter()
        one()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return {"value": round(dec["step_bytes"] / med / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port", "ms_per_step": round(med * 1e3, 1),
            "sample": f"{len(times)} CPU forwards of the full M=1 layer (7 linears, bf16 dequant + F.linear, "
                      f"median); os.cpu_count()={os.cpu_count()}",
            "cpu": _cpu_model()}


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--copies", type=int, default=10)
    ap.add_argument("--prefill-steps", type=int, default=6)
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--kernel-reps", type=int, default=10)
    ap.add_argument("--ungrouped", action="store_true", help="one launch per linear (7 per step)")
    ap.add_argument("--no-quantize", action="store_true")
    ap.add_argument("--no-decode70b", action="store_true")
    ap.add_argument("--quantize-reps", type=int, default=3)
    ap.add_argument("--copy-calib", action="store_true", help="only run the plain-copy PMC calibration")
    ap.add_argument("--prefill-only", action="store_true", help="only the prefill lines (for counter runs)")
    ap.add_argument("--decode-counters", action="store_true",
                    help="only eager M=1 decode launches of three layers (for counter runs)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build targets a single MI355X and has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    import tensorshrink_amd  # noqa: F401  (fails loudly without the built library)
    torch.cuda.set_device(0)
    if args.copy_calib:
        copy_calibration()
        return
    if args.decode_counters:
        decode_counter_launches()
        return
    if args.prefill_only:
        pre = bench_prefill(args)
        pre["short_prompt"] = bench_prefill_short(args)
        print(json.dumps({"prefill": pre}), flush=True)
        return
    import recipes
    opts = dict(bits=4, group_size=128, outlier_frac=0.001, double_quant=True, nf_quant=True)
    log("decode: building layers")
    copies = build_copies(recipes.LLAMA3_8B_LINEARS, lambda name: opts, args.copies)
    dec = bench_decode(args, recipes.LLAMA3_8B_LINEARS, lambda name: opts, args.copies, args.steps, args.warmup,
                       args.kernel_reps, copies=copies)
    kern = dec["kern"]
    # the drop-in path: one QuantLinear.forward per linear, 7 launches a step
    alt_units = GROUPED_UNITS if args.ungrouped else SINGLE_UNITS
    alt = bench_decode(args, recipes.LLAMA3_8B_LINEARS, lambda name: opts, args.copies, min(args.steps, 30),
                       min(args.warmup, 10), args.kernel_reps, copies=copies, units=alt_units)
    alt_line = {"launches_per_step": len(alt_units), "us_per_step": round(alt["ms_per_step"] * 1e3, 2),
                "GBps": round(alt["value"], 1), "frac_of_hbm_peak": round(alt["value"] / HBM_PEAK_GBS, 4),
                "step_gpu_us": round(alt["step_gpu_us"], 2), "per_launch_isolated": alt["kern"],
                "traffic": (load_traffic(alt_units) or {}).get("bytes_per_step")}
    log(f"decode ({len(alt_units)} launches/step): {alt_line['us_per_step']} us/step, {alt_line['GBps']} GB/s")
    # the 4096x4096 4-bit NF4 + DQ linear by itself (the
    # layer's q), M = 1 and 16, with the reference CPU fallback beside it
    cfg1 = {"workload": "BASELINE config 1: single QuantLinear 4096x4096, 4-bit NF4 + double quant, group 128, "
                        "outlier_frac 0.001; one launch per forward, 10 rotating copies",
            "lines": [bench_single(copies, 0, M, args.kernel_reps * 3) for M in (1, 16)]}
    if not args.no_cpu:
        for line in cfg1["lines"]:
            line["cpu_baseline"] = cpu_forward_baseline(copies[0][0][1], line["M"], min(args.cpu_budget, 8.0))
    log(f"cfg1: {cfg1['lines']}")
    cfg2 = bench_cfg2(args)
    log(f"cfg2: {cfg2['lines']}")
    k_us = sum(v["us"] for v in kern.values())
    achieved = dec["step_bytes"] / (dec["step_gpu_us"] * 1e-6) / 1e9
    log(f"decode: {dec['ms_per_step'] * 1e3:.1f} us/step, {dec['value']:.0f} GB/s; GPU {dec['step_gpu_us']:.1f} "
        f"us/step -> {achieved:.0f} GB/s; isolated launches (resident x) {k_us:.1f} us/layer")
    traffic = load_traffic(dec["units"])
    d70 = None
    if not args.no_decode70b:
        log("decode 70B (config 5): building layers")
        d70r = bench_decode(args, recipes.LLAMA3_70B_LINEARS, lambda name: CFG5_OPTS[name], 3, 15, 3, 3,
                            sigma=0.015, seed0=5100)
        d70 = {"workload": "decode M=1, Llama-3-70B-shaped layer, BASELINE config 5 mix: q/k/v/o 8-bit NF8 + DQ, "
                           "gate/up 4-bit NF4 + DQ (group 128), down 2-bit companded + DQ (group 64); 3 rotating "
                           "copies; 4 launches per step",
               "bytes_per_step": d70r["step_bytes"], "us_per_step": round(d70r["ms_per_step"] * 1e3, 2),
               "GBps": round(d70r["value"], 1), "frac_of_hbm_peak": round(d70r["value"] / HBM_PEAK_GBS, 4),
               "step_gpu_us": round(d70r["step_gpu_us"], 2),
               "per_launch_isolated": d70r["kern"]}
        log(f"decode 70B: {d70['us_per_step']} us/step, {d70['GBps']} GB/s")
        del d70r
        torch.cuda.empty_cache()
    pre = None
    if not args.no_prefill:
        log("prefill: M=2048")
        pre = bench_prefill(args)
        log(f"prefill: {pre}")
        log("prefill: short prompt (M=256)")
        pre["short_prompt"] = bench_prefill_short(args)
        log(f"prefill short prompt: {pre['short_prompt']}")
    quant = None
    if not args.no_quantize:
        log("quantize: 28672x8192")
        quant = bench_quantize(args)
        log(f"quantize: {quant}")
        quant["module"] = bench_quantize_module(args)
        log(f"quantize_module: {quant['module']}")
    cpu = None
    if not args.no_cpu:
        log("cpu baseline")
        cpu = cpu_baseline(dec, args.cpu_budget)
        log(f"cpu baseline: {cpu}")
    out = {
        "metric": "QuantLinear M=1 HBM GB/s (% peak); M=2048 TFLOPS (% MFMA peak)",
        "value": round(dec["value"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 activations x 4-bit codes, fp32 accumulate",
        "data": "synthetic: seeded N(0,0.02) fp16 weights with 0.1% x20 outliers, N(0,1) bf16 activations",
        "config": {"workload": "decode M=1, Llama-3-8B-shaped layer (q,k,v,o,gate,up,down), 4-bit NF4 + double "
                               "quant, group 128, outlier_frac 0.001 (BASELINE config 3); 10 rotating copies; "
                               + ("7 launches per step" if args.ungrouped else
                                  "4 launches per step (q/k/v and gate/up grouped)"),
                   "M": 1, "bytes_per_step": dec["step_bytes"], "frac_of_hbm_peak": round(dec["value"] / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic["bytes_per_step"] if traffic else None,
                     "kernel": "ts::decode_kernel (4-bit NF4 + DQ, group 128, bf16), the only kernel of a "
                               "step; achieved = algorithmic bytes of a step's launches / their GPU time (HIP "
                               "events on the launch stream around each replay of the timed region, per step); "
                               "traffic = HBM bytes of those launches (PMC)",
                     "step_gpu_us": round(dec["step_gpu_us"], 2),
                     "isolated_launch_us_per_layer": round(k_us, 2),
                     "per_launch_isolated": kern,
                     "traffic_per_launch": traffic["per_launch_bytes"] if traffic else None},
        "decode_drop_in" if not args.ungrouped else "decode_grouped": alt_line,
        "cfg1": cfg1,
        "cfg2": cfg2,
        "decode_cfg5": d70,
        "prefill": pre,
        "quantize": quant,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
