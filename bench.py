#!/usr/bin/env python3
"""Benchmark of the int4 MatMulNBits / int8 dynamic-quant path on one MI355X.

Headline (the JSON line's "value"): the decode-shape MatMulNBits GEMV,
M=1, K=N=4096, block 128, symmetric, in GB/s of algorithmic traffic
(K*N/2 + N*ceil(K/bs)*4 + M*K*4 + M*N*4 bytes per call).  One step is one
pass of the operator over one batch of synthetic weights: a call on each of
P distinct weight packs (P = 38 at the headline, > 300 MB, more than the
256 MB Infinity Cache, so every call streams its weights from HBM).  A step
is recorded once as a HIP graph; --warmup replays run untimed, then exactly
--steps replays are timed between device synchronisations with HIP events
on the library's stream (the stream the kernels run on).

Also reported (extra keys on the same line):
  roofline      the GEMV kernel: algorithmic bytes per launch / its average
                launch duration over the timed region (timed region / launches,
                every launch in it being that kernel); the per-dispatch event
                duration is listed beside it
  cpu_baseline  the oracle (a C restatement of the reference's Dart
                algorithm) on the host: the headline call, plus legs for the
                single-node config, the M=512 prefill GEMM and the int8 chain
                (one warmup, then min and mean over the timed calls)
  gemm          prefill GEMM M=512, K=N=4096, block 32 with zero points:
                TFLOP/s and its MFMA roofline
  int8          DynamicQuantizeLinear [512,1024] -> MatMulInteger
                [1024,3072] -> fp32 rescale
  decode_sweep  M in {1,4,8} x the four decode projections, block 128
  decoder       end-to-end Qwen3-0.6B-shaped int4 decoder: 256-token prefill
                and 64 greedy decode steps, tokens/s

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]
"""
import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_FP16_PEAK_TFLOPS = 2500.0
MFMA_FP32_PEAK_TFLOPS = 157.3
INT8_PEAK_TOPS = 5000.0
ROTATE_BYTES = 320 * 1024 * 1024
HOST_CPU_SHARE = 16  # host cores a single-GPU MI355X node allots to one GPU's jobs
TRAFFIC_SOURCE = ("committed rocprofv3 counter passes (FETCH_SIZE, WRITE_SIZE) of the same "
                  "workload, profiles/traffic.json; not measured in this run")


def mmnb_bytes(m, k, n, bs, zp):
    nb = (k + bs - 1) // bs
    b = k * n // 2 + n * nb * 4 + m * k * 4 + m * n * 4
    if zp:
        b += n * ((nb + 1) // 2)
    return b


def make_packs(ctx, ops, synth, m, k, n, bs, zp, count, seed):
    packs = []
    for i in range(count):
        b_q, scales, zps = synth.mmnb_weights(k, n, bs, zp, seed * 100 + i,
                                              (0.002, 0.02) if not zp else (0.005, 0.02))
        packs.append(ops.pack_nbits(b_q, scales, zps, k=k, n=n, bits=4, block_size=bs,
                                    ctx=ctx))
    return packs


def time_mmnb(ctx, lib, packs, da, m, dy, steps, warmup, min_calls=32, min_dispatches=200):
    """One step = one call on each pack.  Each HIP graph holds enough whole
    steps for at least min_calls calls (one step for the headline's 38
    packs), so the gap between graph launches is amortised like the gap
    between kernels; `steps` steps are timed (rounded up to whole graphs).
    Then two eager passes with start/end timestamps taken by each dispatch
    (the per-kernel durations a kernel tracer reports): `queued`, at least
    min_dispatches calls enqueued without waiting, and `isolated`,
    min_dispatches calls each launched after the previous one finished.
    Returns (timed steps, ms per step, ms per call, queued, isolated), the
    last two as {kernel: per-dispatch durations in ms}."""
    P = len(packs)
    per_graph = max(1, -(-min_calls // P))  # steps per graph

    def issue_round():
        for p in packs:
            lib.check(ctx.lib.mmnb_matmul_nbits_dev(ctx.handle, p.handle, da.ptr, m, dy.ptr))

    issue_round()  # sizes any scratch before capture
    ctx.synchronize()
    ctx.graph_begin()
    for _ in range(per_graph):
        issue_round()
    g = ctx.graph_end()
    launches = -(-steps // per_graph)
    steps = launches * per_graph
    for _ in range(-(-warmup // per_graph)):
        ctx.graph_launch(g)
    ctx.synchronize()
    ctx.event_record(0)
    for _ in range(launches):
        ctx.graph_launch(g)
    ctx.event_record(1)
    ctx.synchronize()
    total_ms = ctx.event_elapsed_ms(0, 1)
    ctx.graph_destroy(g)
    # eager pass: one dispatch per call, each timed by its own start/end
    # timestamps (these include a fixed per-dispatch cost that back-to-back
    # graph launches do not pay)
    nk = max(min_dispatches, min(steps * P, 2048))
    ctx.kernel_timing(True, max_launches=4 * nk)
    done = 0
    while done < nk:
        issue_round()
        done += P
    kt = ctx.kernel_timing_read()
    queued = {name: ctx.kernel_timing_samples(name) for name in kt}
    ctx.kernel_timing(False)
    # isolated pass: each call launched on an idle GPU (the host waits for the
    # previous one to finish), the regime a kernel tracer puts every dispatch in
    ctx.kernel_timing(True, max_launches=4 * min_dispatches)
    for i in range(min_dispatches):
        lib.check(ctx.lib.mmnb_matmul_nbits_dev(ctx.handle, packs[i % P].handle, da.ptr, m,
                                                dy.ptr))
        ctx.synchronize()
    kt = ctx.kernel_timing_read()
    isolated = {name: ctx.kernel_timing_samples(name) for name in kt}
    ctx.kernel_timing(False)
    return steps, total_ms / steps, total_ms / (steps * P), queued, isolated


def dispatch_stats(ms):
    """Median / mean / min / max (µs) and count of per-dispatch durations."""
    us = np.asarray(ms, np.float64) * 1e3
    return {"count": int(us.size), "median_us": float(np.median(us)),
            "mean_us": float(us.mean()), "min_us": float(us.min()), "max_us": float(us.max())}


def bench_gemv(ctx, lib, ops, synth, m, k, n, bs, zp, steps, warmup, seed=1):
    """GB/s of one GEMV shape over rotated weight packs.  `gbs` / `sustained_*`
    are the back-to-back rate (graph replays: timed region / calls);
    `dispatch` holds the per-dispatch durations of the GEMV kernel launched on
    an idle GPU (median over 200 isolated launches), the figure a kernel trace
    reproduces; `queued_dispatch` the same kernel's durations when launches
    are enqueued without waiting."""
    per_call = mmnb_bytes(m, k, n, bs, zp)
    count = max(2, int(np.ceil(ROTATE_BYTES / (k * n // 2 + n * ((k + bs - 1) // bs) * 4))))
    packs = make_packs(ctx, ops, synth, m, k, n, bs, zp, count, seed)
    a = synth.activations(m, k, seed)
    da = ctx.to_device(a)
    dy = ctx.alloc(m * n * 4)
    n_steps, ms_step, ms_call, queued, isolated = time_mmnb(ctx, lib, packs, da, m, dy, steps,
                                                            warmup)
    kname = "k_gemv_valu" if "k_gemv_valu" in isolated else sorted(isolated)[0]
    disp = dispatch_stats(isolated[kname])
    res = {"m": m, "k": k, "n": n, "block": bs, "zero_points": zp, "packs": count,
           "bytes_per_call": per_call, "bytes_per_step": per_call * count,
           "steps": n_steps, "calls": n_steps * count, "ms_per_step": ms_step,
           "ms_per_call": ms_call, "gbs": per_call / (ms_call * 1e-3) / 1e9, "kernel": kname,
           "sustained_us": ms_call * 1e3, "sustained_gbs": per_call / (ms_call * 1e-3) / 1e9,
           "dispatch": disp,
           "dispatch_gbs": per_call / (disp["median_us"] * 1e-6) / 1e9,
           "queued_dispatch": dispatch_stats(queued[kname]),
           "kernels": {k_: dispatch_stats(v) for k_, v in isolated.items()}}
    da.free()
    dy.free()
    for p in packs:
        p.free()
    return res


def bench_gemm(ctx, lib, ops, synth, m, k, n, bs, zp, steps, warmup):
    """Prefill MatMulNBits: the op back to back (graph replays: `k_prep_a` +
    the GEMM per call) and per-dispatch durations of each kernel, queued
    (calls enqueued without waiting) and isolated (each launched on an idle
    GPU).  The roofline is the GEMM kernel's median queued dispatch, the
    back-to-back regime of the headline's roofline (the graph's timed region
    holds the prep kernel too, so the kernel's own share comes from its
    dispatch timestamps); `op` gives what a caller sees: the prep kernel's
    median added to the GEMM's, and the back-to-back rate of whole calls."""
    p = synth.mmnb_problem(m, k, n, bs, zp, seed=2, outlier_frac=0.01)
    pack = ops.pack_nbits(p.b_q, p.scales, p.zero_points, k=k, n=n, bits=4, block_size=bs,
                          ctx=ctx)
    da = ctx.to_device(p.a)
    dy = ctx.alloc(m * n * 4)
    n_steps, _, ms_step, queued, isolated = time_mmnb(ctx, lib, [pack], da, m, dy, steps,
                                                      warmup)
    flops = 2.0 * m * k * n
    g = dispatch_stats(isolated["k_gemm_mfma"])
    gq = dispatch_stats(queued["k_gemm_mfma"])
    pr = dispatch_stats(isolated["k_prep_a"]) if "k_prep_a" in isolated else None
    achieved = flops / (gq["median_us"] * 1e-6) / 1e12
    op_us = g["median_us"] + (pr["median_us"] if pr else 0.0)
    res = {"m": m, "k": k, "n": n, "block": bs, "zero_points": zp, "steps": n_steps,
           "ms_per_call": ms_step, "tflops": flops / (ms_step * 1e-3) / 1e12,
           "gemm_dispatch": g, "prep_dispatch": pr,
           "gemm_queued_dispatch": gq,
           "op": {"dispatch_us": op_us, "dispatch_tflops": flops / (op_us * 1e-6) / 1e12,
                  "sustained_us": ms_step * 1e3,
                  "sustained_tflops": flops / (ms_step * 1e-3) / 1e12},
           "roofline": {"bound": "mfma", "achieved": achieved,
                        "peak": MFMA_FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                        "frac": achieved / MFMA_FP16_PEAK_TFLOPS,
                        "kernel": "k_gemm_mfma",
                        "timing": "median of the GEMM kernel's per-dispatch start/end "
                                  "timestamps, calls enqueued back to back",
                        "kernel_median_us": gq["median_us"], "dispatches": gq["count"],
                        "isolated_median_us": g["median_us"],
                        "isolated_achieved": flops / (g["median_us"] * 1e-6) / 1e12,
                        "mfma_passes": 2,
                        "mfma_utilisation": 2 * achieved / MFMA_FP16_PEAK_TFLOPS,
                        "vs_fp32_mfma_peak": achieved / MFMA_FP32_PEAK_TFLOPS}}
    if (m, k, n, bs, zp) == (512, 4096, 4096, 32, True):
        tr = measured_traffic("gemm_m512_k4096_n4096_bs32_zp")
        res["roofline"]["traffic"] = tr
        res["roofline"]["traffic_source"] = TRAFFIC_SOURCE if tr else None
    else:
        res["roofline"]["traffic"] = None
    da.free()
    dy.free()
    pack.free()
    return res


def _graph_us(ctx, fn, steps, warmup, per_graph=20):
    """Per-call time of fn: a HIP graph of per_graph calls, warmup untimed
    replays, then `steps` replays timed with events on the library stream."""
    fn()
    ctx.synchronize()
    ctx.graph_begin()
    for _ in range(per_graph):
        fn()
    g = ctx.graph_end()
    for _ in range(warmup):
        ctx.graph_launch(g)
    ctx.synchronize()
    ctx.event_record(0)
    for _ in range(steps):
        ctx.graph_launch(g)
    ctx.event_record(1)
    ctx.synchronize()
    us = ctx.event_elapsed_ms(0, 1) * 1e3 / (steps * per_graph)
    ctx.graph_destroy(g)
    return us


def bench_int8(ctx, lib, ops, synth, steps, warmup):
    """The int8 chain DQL [512,1024] -> MatMulInteger [1024,3072] -> rescale,
    with the exact int32 accumulator also written (the MatMulInteger node's
    own output kept) and fused (d_acc NULL: only the fp32 result leaves the
    kernel, as in the graph where the int32 tensor feeds Cast -> Mul alone);
    and its two ops alone (DQL; MatMulInteger with the int32 output, the
    operator's own result).  Per-call times from graphs of 20 calls."""
    m, k, n = 512, 1024, 3072
    x, b = synth.int8_chain_problem(m, k, n)
    pack = ops.pack_integer(b, np.array(0, np.int8), ctx=ctx)
    bscale = np.array([0.01], np.float32)
    dx, dbs = ctx.to_device(x), ctx.to_device(bscale)
    daq, dsc, dzp = ctx.alloc(m * k), ctx.alloc(4), ctx.alloc(4)
    dacc, dy = ctx.alloc(m * n * 4), ctx.alloc(m * n * 4)

    def chain(acc_ptr):
        lib.check(ctx.lib.mmnb_dynamic_matmul_dev(ctx.handle, pack.handle, dx.ptr, m, dbs.ptr, 1,
                                                  daq.ptr, dsc.ptr, dzp.ptr, acc_ptr, dy.ptr))

    def dql():
        lib.check(ctx.lib.mmnb_dynamic_quantize_linear_dev(ctx.handle, dx.ptr, m * k, daq.ptr,
                                                           dsc.ptr, dzp.ptr))

    def mmi():
        lib.check(ctx.lib.mmnb_matmul_integer_dev(ctx.handle, pack.handle, daq.ptr, 0, 1, m,
                                                  dzp.ptr, 1, dacc.ptr))

    chain_us = _graph_us(ctx, lambda: chain(dacc.ptr), steps, warmup)
    fused_us = _graph_us(ctx, lambda: chain(None), steps, warmup)
    dql_us = _graph_us(ctx, dql, steps, warmup)
    mmi_us = _graph_us(ctx, mmi, steps, warmup)
    mmi_bytes = m * k + k * n + 4 * m * n          # A u8, B i8, int32 out
    dql_bytes = 4 * m * k + m * k
    res = {"m": m, "k": k, "n": n, "ms_per_chain": chain_us * 1e-3,
           "fused": {"ms_per_chain": fused_us * 1e-3},
           "dql_us": dql_us, "dql_gbs": dql_bytes / (dql_us * 1e-6) / 1e9,
           "mmi_us": mmi_us,
           "mmi_roofline": {"bound": "hbm", "achieved": mmi_bytes / (mmi_us * 1e-6) / 1e9,
                            "peak": HBM_PEAK_GBS, "unit": "GB/s",
                            "frac": mmi_bytes / (mmi_us * 1e-6) / 1e9 / HBM_PEAK_GBS,
                            "tops": 2.0 * m * k * n / (mmi_us * 1e-6) / 1e12,
                            "int8_peak_frac": 2.0 * m * k * n / (mmi_us * 1e-6) / 1e12
                            / INT8_PEAK_TOPS}}
    for bf in (dx, dbs, daq, dsc, dzp, dacc, dy):
        bf.free()
    pack.free()
    return res


def _kernel_us_per_call(kt, reps):
    """{kernel: µs per call} and the sum, from a timing read over `reps` calls."""
    per = {name: v[1] / reps * 1e3 for name, v in kt.items()}
    return per, sum(per.values())


def bench_qlinear(ctx, lib, ops, reps=200):
    """QLinearMatMul at the int8 chain's shape ([512,1024] u8 x [1024,3072]
    i8 -> u8) and a ResNet-50 layer-1 3x3 convolution (1x64x56x56 u8,
    64x64x3x3 i8, pad 1) as ConvInteger (int32 out) and QLinearConv
    (per-channel scales, bias, u8 out).  Kernel times from dispatch events
    (each includes the dispatch's own start-up, ~4 us for an empty kernel);
    QLinearMatMul and ConvInteger also back to back in graphs of 20 calls
    (QLinearConv uploads its per-channel parameters and is not captured)."""
    out = {}
    rng = np.random.default_rng(7)
    m, k, n = 512, 1024, 3072
    a = rng.integers(0, 256, (m, k)).astype(np.uint8)
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    pack = ops.pack_integer(b, np.int8(0), ctx)
    da, dz, dq = ctx.to_device(a), ctx.to_device(np.array([128], np.int32)), ctx.alloc(m * n)

    def qmm():
        lib.check(ctx.lib.mmnb_qlinear_matmul_dev(ctx.handle, pack.handle, da.ptr, 0, 1, m,
                                                  dz.ptr, 1, 0.02, 0.01, 0.5, 3, 0, dq.ptr))
    for _ in range(10):
        qmm()
    ctx.kernel_timing(True, max_launches=2 * reps)
    for _ in range(reps):
        qmm()
    per, tot = _kernel_us_per_call(ctx.kernel_timing_read(), reps)
    ctx.kernel_timing(False)
    nbytes = m * k + k * n + m * n
    out["qlinear_matmul"] = {
        "m": m, "k": k, "n": n, "kernels_us": per, "us_per_call": tot,
        "back_to_back_us": _graph_us(ctx, qmm, 50, 5),
        "gbs": nbytes / (tot * 1e-6) / 1e9, "hbm_frac": nbytes / (tot * 1e-6) / 1e9 / HBM_PEAK_GBS,
        "tops": 2.0 * m * k * n / (tot * 1e-6) / 1e12}
    for bf in (da, dz, dq):
        bf.free()
    pack.free()
    # convolution, ResNet-50 layer 1 (3x3, 64 -> 64, 56x56, pad 1)
    c, h, w, mo = 64, 56, 56, 64
    x = rng.integers(0, 256, (1, c, h, w)).astype(np.uint8)
    wt = rng.integers(-127, 128, (mo, c, 3, 3)).astype(np.int8)
    cp = ops.pack_conv(wt, np.zeros(mo, np.int8), 1, ctx)
    prm = lib.ConvParams()
    prm.strides[0] = prm.strides[1] = 1
    prm.dilations[0] = prm.dilations[1] = 1
    for i in range(4):
        prm.pads[i] = 1
    dx, dy32, dy8 = ctx.to_device(x), ctx.alloc(mo * h * w * 4), ctx.alloc(mo * h * w)
    ws = rng.uniform(0.001, 0.01, mo).astype(np.float32)
    bias = rng.integers(-1000, 1000, mo).astype(np.int32)

    def conv():
        lib.check(ctx.lib.mmnb_conv_integer_dev(ctx.handle, cp.handle, dx.ptr, 0, 1, c, h, w, 128,
                                                ctypes.byref(prm), dy32.ptr))

    def qconv():
        lib.check(ctx.lib.mmnb_qlinear_conv_dev(
            ctx.handle, cp.handle, dx.ptr, 0, 1, c, h, w, 128, 0.02, ws.ctypes.data, mo, 0.05,
            128, 0, bias.ctypes.data, ctypes.byref(prm), dy8.ptr))
    ops_ = 2.0 * mo * h * w * c * 9
    for name, fn, obytes in (("conv_integer", conv, 4), ("qlinear_conv", qconv, 1)):
        for _ in range(5):
            fn()
        ctx.kernel_timing(True, max_launches=4 * reps)
        for _ in range(reps):
            fn()
        per, tot = _kernel_us_per_call(ctx.kernel_timing_read(), reps)
        ctx.kernel_timing(False)
        nbytes = c * h * w + mo * c * 9 + mo * h * w * obytes
        out[name] = {"shape": "x 1x64x56x56 u8, w 64x64x3x3 i8, pad 1", "kernels_us": per,
                     "us_per_call": tot, "tops": ops_ / (tot * 1e-6) / 1e12,
                     "gbs": nbytes / (tot * 1e-6) / 1e9}
        if fn is conv:
            out[name]["back_to_back_us"] = _graph_us(ctx, conv, 50, 5)
    for bf in (dx, dy32, dy8):
        bf.free()
    cp.free()
    return out


def bench_nbits_ex(ctx, lib, ops, reps=300):
    """MatMulNBits with the inputs the reference rejects, at the headline
    decode shape M=1, K=N=4096, block 128: bits 8 (uint8 zero points),
    float zero points, act-order g_idx, bias.  Per-call kernel time (the
    4-bit kernels plus the gather / block-sum / correction launches) and
    GB/s over the operator's own bytes."""
    out = {}
    rng = np.random.default_rng(9)
    k = n = 4096
    bs, m = 128, 1
    nb = k // bs
    a = rng.standard_normal((m, k)).astype(np.float32)
    da, dy = ctx.to_device(a), ctx.alloc(m * n * 4)
    cases = {
        "bits8_u8zp": dict(bits=8, z=rng.integers(0, 256, n * nb).astype(np.uint8)),
        "bits4_float_zp": dict(bits=4, z=rng.uniform(0, 15, (n, nb)).astype(np.float32)),
        "bits4_g_idx": dict(bits=4, g=rng.permutation(np.repeat(np.arange(nb), bs))),
        "bits4_bias": dict(bits=4, bias=rng.standard_normal(n).astype(np.float32)),
    }
    for name, cfg in cases.items():
        bits = cfg["bits"]
        bq = rng.integers(0, 256, (n, nb, bs * bits // 8)).astype(np.uint8)
        sc = rng.uniform(0.002, 0.02, n * nb).astype(np.float32)
        pack = ops.pack_nbits_ex(bq, sc, cfg.get("z"), cfg.get("g"), cfg.get("bias"), k=k, n=n,
                                 bits=bits, block_size=bs, ctx=ctx)

        def call():
            lib.check(ctx.lib.mmnb_matmul_nbits_dev(ctx.handle, pack.handle, da.ptr, m, dy.ptr))
        for _ in range(10):
            call()
        ctx.kernel_timing(True, max_launches=5 * reps)
        for _ in range(reps):
            call()
        per, tot = _kernel_us_per_call(ctx.kernel_timing_read(), reps)
        ctx.kernel_timing(False)
        z = cfg.get("z")
        nbytes = (bq.nbytes + sc.nbytes + (0 if z is None else z.nbytes) + a.nbytes + m * n * 4
                  + (0 if cfg.get("g") is None else k * 4)
                  + (0 if cfg.get("bias") is None else n * 4))
        out[name] = {"m": m, "k": k, "n": n, "block": bs, "bits": bits, "kernels_us": per,
                     "us_per_call": tot, "bytes": nbytes, "gbs": nbytes / (tot * 1e-6) / 1e9}
        pack.free()
    da.free()
    dy.free()
    return out


def bench_decoder(ctx, lib, runs=3):
    """The end-to-end synthetic decoder (Qwen3-0.6B shape: 28 layers, hidden
    1024, 16/8 heads of 128, SwiGLU 3072, vocab 151936, random int4 weights,
    block 128): 256-token prefill, then 64 greedy decode steps, every
    MatMulNBits on the GPU.  Best of `runs` (the first untimed run also
    records the decode-step graph)."""
    from onnx_runtime_dart_amd import decoder as G

    cfg = G.QWEN3_0_6B
    w = G.random_weights(cfg, seed=0)
    dec = G.GpuDecoder(w, ctx)
    prompt = np.random.default_rng(3).integers(0, cfg.vocab, 256)
    steps = 64
    try:
        dec.prefill(prompt)
        dec.decode(steps)
        best = None
        for _ in range(runs):
            dec.reset()
            ctx.synchronize()
            t0 = time.perf_counter()
            dec.prefill(prompt)
            t1 = time.perf_counter()
            dec.decode(steps)
            t2 = time.perf_counter()
            r = (t1 - t0, t2 - t1)
            if best is None or sum(r) < sum(best):
                best = r
    finally:
        dec.free()
    pf, dc = best
    per_tok = cfg.weight_bytes_per_token()
    return {"config": "Qwen3-0.6B shape, 28 layers, int4 block 128, random weights",
            "prefill_tokens": 256, "decode_steps": steps,
            "prefill_ms": pf * 1e3, "decode_ms": dc * 1e3,
            "prefill_tok_s": 256 / pf, "decode_tok_s": steps / dc,
            "e2e_tok_s": (256 + steps) / (pf + dc),
            "decode_ms_per_token": dc * 1e3 / steps,
            "weight_bytes_per_token": per_tok,
            "decode_weight_gbs": per_tok * steps / dc / 1e9,
            "launches_per_token": 5 * cfg.layers + 3}


def bench_platform(ctx, lib):
    """Per-dispatch floor and streaming-read ceiling of this GPU, measured
    with the library's calibration kernels and the same dispatch events."""
    out = {}
    # empty kernel of 1..1024 workgroups of 256 threads: duration from its
    # dispatch events, and the per-launch cost inside a graph of 100 launches
    sweep = {}
    for blocks in (1, 64, 256, 512, 1024):
        ctx.kernel_timing(True, max_launches=400)
        for _ in range(200):
            lib.check(ctx.lib.mmnb_probe_empty(ctx.handle, blocks))
        kt = ctx.kernel_timing_read()
        ctx.kernel_timing(False)
        ev = kt["k_probe_empty"][1] / kt["k_probe_empty"][0] * 1e3
        g_us = _graph_us(ctx, lambda: lib.check(ctx.lib.mmnb_probe_empty(ctx.handle, blocks)),
                         steps=20, warmup=2, per_graph=100)
        sweep[str(blocks)] = {"dispatch_event_us": ev, "in_graph_us": g_us}
    out["empty_kernel_sweep"] = sweep
    out["empty_kernel_us"] = sweep["1024"]["dispatch_event_us"]
    for label, size, nbuf, reps in (("read_8.95MB", 8945664, 37, 370),
                                    ("read_134MB", 134217728, 3, 30)):
        bufs = [ctx.alloc(size) for _ in range(nbuf)]
        for b in bufs:
            lib.check(ctx.lib.mmnb_memset_dev(ctx.handle, b.ptr, 1, size))
        for b in bufs:  # warm
            lib.check(ctx.lib.mmnb_probe_stream_read(ctx.handle, b.ptr, size))
        ctx.kernel_timing(True, max_launches=2 * reps)
        for i in range(reps):
            lib.check(ctx.lib.mmnb_probe_stream_read(ctx.handle, bufs[i % nbuf].ptr, size))
        kt = ctx.kernel_timing_read()
        ctx.kernel_timing(False)
        us = kt["k_probe_read"][1] / kt["k_probe_read"][0] * 1e3
        # back-to-back rate: graph of one rotation, events around the replays
        ctx.synchronize()
        ctx.graph_begin()
        for b in bufs:
            lib.check(ctx.lib.mmnb_probe_stream_read(ctx.handle, b.ptr, size))
        g = ctx.graph_end()
        ctx.graph_launch(g)
        ctx.synchronize()
        ctx.event_record(0)
        for _ in range(max(1, reps // nbuf)):
            ctx.graph_launch(g)
        ctx.event_record(1)
        ctx.synchronize()
        b2b = ctx.event_elapsed_ms(0, 1) * 1e3 / (max(1, reps // nbuf) * nbuf)
        ctx.graph_destroy(g)
        out[label] = {"kernel_us": us, "kernel_gbs": size / (us * 1e-6) / 1e9,
                      "back_to_back_us": b2b, "back_to_back_gbs": size / (b2b * 1e-6) / 1e9}
        for b in bufs:
            b.free()
    return out


def measured_traffic(workload):
    """HBM bytes per launch from the committed rocprofv3 counter summary
    (FETCH_SIZE and WRITE_SIZE per dispatch, each scaled by what the counter
    reads for a copy of known size), or None if not measured."""
    path = ROOT / "profiles" / "traffic.json"
    try:
        return json.loads(path.read_text()).get(workload, {}).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def _time_cpu(fn, budget_s, min_iters=2):
    """tool/bench.dart's method: one untimed warmup call, then timed calls
    until the budget is spent (at least min_iters); (min, mean, count) in s."""
    fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < min_iters:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return min(times), float(np.mean(times)), len(times)


def cpu_baseline(synth, budget_s):
    """The oracle (C restatement of the reference's Dart arithmetic) timed on
    this host.  MatMulNBits dequantises to a fresh K x N fp32 buffer, then
    runs the sequential-k fp32 GEMV/GEMM; the reference runs it on one
    isolate (its pool never takes MatMulNBits, onnx_graph.dart:578-614), so
    the headline figure is single-threaded.  Legs: the headline column-sliced
    over the host threads (context), the single-node config,
    the M=512 prefill GEMM (all host threads, column-sliced like the pool's
    partition, plus one thread on a 16-row sample) and the int8 chain
    (DynamicQuantizeLinear -> MatMulInteger -> rescale, one thread)."""
    from oracle import refcpu

    # A single-GPU MI355X node gives each GPU's jobs a share of 16 host cores,
    # whatever the machine's own count: the multi-threaded legs use that share (or fewer
    # if fewer CPUs are allowed to this process), and both counts are stated.
    nproc = os.cpu_count() or 1
    allowed = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else nproc
    threads = min(HOST_CPU_SHARE, allowed, refcpu.host_threads())
    # headline: M=1 K=N=4096 block 128, symmetric
    m, k, n, bs = 1, 4096, 4096, 128
    p = synth.mmnb_problem(m, k, n, bs, False, seed=1, scale_range=(0.002, 0.02))
    lo, mean, cnt = _time_cpu(lambda: refcpu.matmul_nbits(p.a, p.b_q, p.scales, None, k, n, 4,
                                                          bs), 0.28 * budget_s)
    per = mmnb_bytes(m, k, n, bs, False)
    out = {"value": per / mean / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
           "sample": f"MatMulNBits M={m} K={k} N={n} block {bs}, no zero points: 1 warmup + "
                     f"{cnt} timed calls, mean {mean * 1e3:.1f} ms, min {lo * 1e3:.1f} ms",
           "min_ms": lo * 1e3, "mean_ms": mean * 1e3}
    legs = {}
    # the same call column-sliced over the host threads (context only: the
    # reference's pool does not take MatMulNBits)
    lo, mean, cnt = _time_cpu(lambda: refcpu.matmul_nbits(p.a, p.b_q, p.scales, None, k, n, 4,
                                                          bs, threads=threads), 0.07 * budget_s)
    legs["headline_threads"] = {"value": per / mean / 1e9, "unit": "GB/s", "cores": threads,
                                "min_ms": lo * 1e3, "mean_ms": mean * 1e3, "calls": cnt}
    # single-node config: M=1 K=N=1024 block 32 with zero points
    p1 = synth.mmnb_problem(1, 1024, 1024, 32, True, seed=0)
    lo, mean, cnt = _time_cpu(lambda: refcpu.matmul_nbits(p1.a, p1.b_q, p1.scales,
                                                          p1.zero_points, 1024, 1024, 4, 32),
                              0.1 * budget_s)
    legs["single_node_m1_k1024_n1024_bs32_zp"] = {
        "value": mmnb_bytes(1, 1024, 1024, 32, True) / mean / 1e9, "unit": "GB/s", "cores": 1,
        "min_ms": lo * 1e3, "mean_ms": mean * 1e3, "calls": cnt}
    # prefill GEMM: M=512 K=N=4096 block 32 with zero points
    pg = synth.mmnb_problem(512, 4096, 4096, 32, True, seed=2, outlier_frac=0.01)
    lo, mean, cnt = _time_cpu(lambda: refcpu.matmul_nbits(pg.a, pg.b_q, pg.scales,
                                                          pg.zero_points, 4096, 4096, 4, 32,
                                                          threads=threads),
                              0.2 * budget_s, min_iters=1)
    flops = 2.0 * 512 * 4096 * 4096
    rows = np.arange(16)
    lo1, mean1, cnt1 = _time_cpu(lambda: refcpu.matmul_nbits(pg.a[rows], pg.b_q, pg.scales,
                                                             pg.zero_points, 4096, 4096, 4, 32),
                                 0.1 * budget_s, min_iters=1)
    legs["prefill_m512_k4096_n4096_bs32_zp"] = {
        "value": flops / mean / 1e12, "unit": "TFLOP/s", "cores": threads,
        "min_ms": lo * 1e3, "mean_ms": mean * 1e3, "calls": cnt,
        "one_thread_16_rows": {"value": 2.0 * 16 * 4096 * 4096 / mean1 / 1e12,
                               "unit": "TFLOP/s", "cores": 1, "min_ms": lo1 * 1e3,
                               "mean_ms": mean1 * 1e3, "calls": cnt1}}
    # int8 chain: DQL [512,1024] -> MatMulInteger [1024,3072] -> fp32 rescale
    x, b = synth.int8_chain_problem(512, 1024, 3072)
    bscale = np.array([0.01], np.float32)

    def chain():
        y, sc, zp = refcpu.dynamic_quantize_linear(x)
        acc = refcpu.matmul_integer(y, b, zp, 0)
        return refcpu.rescale(acc, sc, bscale)

    lo, mean, cnt = _time_cpu(chain, 0.25 * budget_s, min_iters=1)
    legs["int8_chain_m512_k1024_n3072"] = {
        "value": 2.0 * 512 * 1024 * 3072 / mean / 1e12, "unit": "TOP/s", "cores": 1,
        "min_ms": lo * 1e3, "mean_ms": mean * 1e3, "calls": cnt}
    out["legs"] = legs
    out["host"] = {"nproc": nproc, "cpus_allowed": allowed, "cpu_share_per_gpu": HOST_CPU_SHARE,
                   "threads_used_by_multithreaded_legs": threads}
    return out


PROFILE_CALLS = 200
EXTRAS = ["gemv_bs32_zp", "c1_gemv", "gemv_large", "gemm", "int8", "decode_sweep", "qlinear",
          "nbits_ex", "decoder", "platform"]


def profile_calls(ctx, call):
    """The two eager passes of time_mmnb, for a tracer: PROFILE_CALLS calls
    each launched on an idle GPU (the host waits after every call), then
    PROFILE_CALLS calls enqueued without waiting.  No HIP graphs."""
    for i in range(PROFILE_CALLS):
        call(i)
        ctx.synchronize()
    for i in range(PROFILE_CALLS):
        call(i)
    ctx.synchronize()


def profile_pass(ctx, lib, ops, synth, kind):
    """Kernels for a rocprofv3 counter run: one operator workload and a copy
    of known size (the calibration reference for FETCH_SIZE / WRITE_SIZE)."""
    if kind == "gemv":
        m, k, n, bs = 1, 4096, 4096, 128
        count = int(np.ceil(ROTATE_BYTES / (k * n // 2 + n * (k // bs) * 4)))
        packs = make_packs(ctx, ops, synth, m, k, n, bs, False, count, 1)
        da = ctx.to_device(synth.activations(m, k, 1))
        dy = ctx.alloc(m * n * 4)
        profile_calls(ctx, lambda i: lib.check(ctx.lib.mmnb_matmul_nbits_dev(
            ctx.handle, packs[i % count].handle, da.ptr, m, dy.ptr)))
        what = (f"GEMV calls over {count} rotated packs ({mmnb_bytes(m, k, n, bs, False)} "
                f"algorithmic bytes each): {PROFILE_CALLS} isolated, then {PROFILE_CALLS} queued")
    elif kind == "gemv_large":
        # eager dispatches with gaps between them, then graph replays back
        # to back: a kernel trace shows the duration of both
        r = bench_gemv(ctx, lib, ops, synth, 1, 16384, 16384, 128, False, 40, 3, seed=4)
        what = (f"GEMV K=N=16384 block 128: {r['calls']} graph-replayed calls "
                f"({r['ms_per_call'] * 1e3:.2f} us per call) and the eager timing pass "
                f"({r['dispatch']['median_us']:.2f} us median per dispatch)")
        print(f"# profile pass: {what}", file=sys.stderr, flush=True)
        return
    elif kind == "gemm":
        m, k, n, bs = 512, 4096, 4096, 32
        p = synth.mmnb_problem(m, k, n, bs, True, seed=2, outlier_frac=0.01)
        pack = ops.pack_nbits(p.b_q, p.scales, p.zero_points, k=k, n=n, bits=4,
                              block_size=bs, ctx=ctx)
        da = ctx.to_device(p.a)
        dy = ctx.alloc(m * n * 4)
        profile_calls(ctx, lambda i: lib.check(ctx.lib.mmnb_matmul_nbits_dev(
            ctx.handle, pack.handle, da.ptr, m, dy.ptr)))
        what = (f"GEMM calls (M=512 K=N=4096 block 32, zero points; k_prep_a + k_gemm_mfma "
                f"each): {PROFILE_CALLS} isolated, then {PROFILE_CALLS} queued")
    elif kind == "decoder":
        from onnx_runtime_dart_amd import decoder as G
        cfg = G.QWEN3_0_6B
        dec = G.GpuDecoder(G.random_weights(cfg, seed=0), ctx)
        dec.use_graph(False)  # launched one by one, so a tracer sees every kernel
        dec.prefill(np.random.default_rng(3).integers(0, cfg.vocab, 256))
        dec.decode(64)
        ctx.synchronize()
        dec.free()
        what = ("decoder (Qwen3-0.6B shape): 256-token prefill + 64 decode steps, "
                "decode kernels launched eagerly")
    else:
        m, k, n = 512, 1024, 3072
        x, b = synth.int8_chain_problem(m, k, n)
        pack = ops.pack_integer(b, np.array(0, np.int8), ctx=ctx)
        dx, dbs = ctx.to_device(x), ctx.to_device(np.array([0.01], np.float32))
        daq, dsc, dzp = ctx.alloc(m * k), ctx.alloc(4), ctx.alloc(4)
        dacc, dy = ctx.alloc(m * n * 4), ctx.alloc(m * n * 4)
        for _ in range(50):
            lib.check(ctx.lib.mmnb_dynamic_matmul_dev(ctx.handle, pack.handle, dx.ptr, m,
                                                      dbs.ptr, 1, daq.ptr, dsc.ptr, dzp.ptr,
                                                      dacc.ptr, dy.ptr))
        what = "50 int8 chains (DQL [512,1024] -> MatMulInteger [1024,3072] -> rescale)"
    ctx.synchronize()
    nbytes = 64 << 20
    src, dst = ctx.alloc(nbytes), ctx.alloc(nbytes)
    for _ in range(10):
        lib.check(ctx.lib.mmnb_memcpy_d2d(ctx.handle, dst.ptr, src.ptr, nbytes))
    ctx.synchronize()
    print(f"# profile pass: {what}, 10 copies of {nbytes} bytes", file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20,
                    help="timed steps (one step = one call on each rotated weight pack)")
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--quick", action="store_true", help="headline only, no extras")
    ap.add_argument("--extras", default=",".join(EXTRAS),
                    help="comma-separated extra workloads after the headline (default: all "
                         "of " + ",".join(EXTRAS) + ")")
    ap.add_argument("--no-cpu", action="store_true",
                    help="skip the CPU baseline (the line then carries no cpu_baseline)")
    ap.add_argument("--cpu-budget", type=float, default=16.0,
                    help="seconds of host time for the CPU baseline legs")
    ap.add_argument("--profile", action="store_true",
                    help="counter pass for rocprofv3 (prints no JSON): the kernel chosen by "
                         "--profile-kind, then a 64 MiB device-to-device copy (10 calls) as "
                         "the counter calibration")
    ap.add_argument("--profile-kind", default="gemv",
                    choices=["gemv", "gemv_large", "gemm", "int8", "decoder"],
                    help="gemv: headline GEMV, 200 isolated then 200 queued calls over the "
                         "rotated packs; gemv_large: K=N=16384, graph replays and eager "
                         "dispatches; gemm: M=512 K=N=4096 block 32 with zero points, 200 "
                         "isolated then 200 queued calls; int8: the "
                         "DQL -> MatMulInteger -> rescale chain, 50 calls; decoder: the "
                         "Qwen3-shaped decoder, 256-token prefill + 64 steps, eager")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: this build runs the kernel on a single "
              "GPU and has no multi-GPU path; run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    from onnx_runtime_dart_amd import _lib as lib, ops, synth

    ctx = lib.default_context()
    if args.profile:
        profile_pass(ctx, lib, ops, synth, args.profile_kind)
        return
    info = ctx.info()
    print(f"# device {info}", file=sys.stderr, flush=True)

    head = bench_gemv(ctx, lib, ops, synth, 1, 4096, 4096, 128, False, args.steps,
                      args.warmup)
    hd = head["dispatch"]
    print(f"# headline GEMV: {head['gbs']:.0f} GB/s back to back, {head['ms_per_call'] * 1e3:.2f} "
          f"us per call ({head['packs']} calls per step); per dispatch median "
          f"{hd['median_us']:.3f} us over {hd['count']} = {head['dispatch_gbs']:.0f} GB/s",
          file=sys.stderr, flush=True)
    out = {
        "metric": "int4 MatMulNBits GB/s (M=1) & TFLOPS (M=512), % of HBM/MFMA roofline",
        "value": round(head["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4 weights, f32 activations and accumulation",
        "data": "synthetic (seeded): random nibbles and scales, A ~ N(0,1)",
        "config": {"workload": f"MatMulNBits decode GEMV M=1 K=4096 N=4096 block 128, "
                               f"symmetric; one step = one call on each of {head['packs']} "
                               f"distinct weight packs (> 300 MB, streamed from HBM)",
                   "m": 1, "k": 4096, "n": 4096, "block_size": 128, "zero_points": False,
                   "calls_per_step": head["packs"], "bytes_per_call": head["bytes_per_call"],
                   "bytes_per_step": head["bytes_per_step"], "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(head["sustained_gbs"], 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(head["sustained_gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic("gemv_m1_k4096_n4096_bs128"),
                     "traffic_source": TRAFFIC_SOURCE,
                     "kernel": head["kernel"],
                     "timing": "graph replays back to back: timed region (HIP events on the "
                               "launch stream) / launches, the same region as value",
                     "us_per_launch": round(head["sustained_us"], 3),
                     "launches": head["calls"],
                     "dispatch": {"timing": "per-dispatch start/end timestamps (the durations "
                                            "a rocprofv3 kernel trace reports), 200 launches "
                                            "each on an idle GPU",
                                  "median_us": round(hd["median_us"], 3),
                                  "mean_us": round(hd["mean_us"], 3),
                                  "count": hd["count"],
                                  "achieved": round(head["dispatch_gbs"], 1),
                                  "frac": round(head["dispatch_gbs"] / HBM_PEAK_GBS, 4),
                                  "queued_median_us":
                                      round(head["queued_dispatch"]["median_us"], 3)}},
    }
    extras = [] if args.quick else [e for e in args.extras.split(",") if e]
    unknown = [e for e in extras if e not in EXTRAS]
    if unknown:
        print(f"unknown extras {unknown}; choose from {EXTRAS}", file=sys.stderr)
        sys.exit(2)
    try:
        if "gemv_bs32_zp" in extras:
            out["gemv_bs32_zp"] = bench_gemv(ctx, lib, ops, synth, 1, 4096, 4096, 32, True,
                                             args.steps, args.warmup, seed=3)
            print(f"# GEMV bs32+zp: {out['gemv_bs32_zp']['sustained_gbs']:.0f} GB/s back to back",
                  file=sys.stderr, flush=True)
        if "c1_gemv" in extras:
            out["c1_gemv"] = bench_gemv(ctx, lib, ops, synth, 1, 1024, 1024, 32, True, 20, 3,
                                        seed=5)
            print(f"# C1 GEMV M=1 K=N=1024 bs32+zp: {out['c1_gemv']['ms_per_call'] * 1e3:.2f} us "
                  f"per call, {out['c1_gemv']['gbs']:.0f} GB/s", file=sys.stderr, flush=True)
        if "gemv_large" in extras:
            out["gemv_large"] = bench_gemv(ctx, lib, ops, synth, 1, 16384, 16384, 128,
                                           False, 20, 3, seed=4)
            print(f"# GEMV K=N=16384: {out['gemv_large']['sustained_gbs']:.0f} GB/s back to back",
                  file=sys.stderr, flush=True)
        if "gemm" in extras:
            out["gemm"] = bench_gemm(ctx, lib, ops, synth, 512, 4096, 4096, 32, True,
                                     200, 20)
            print(f"# GEMM M=512: {out['gemm']['tflops']:.1f} TFLOP/s op back to back, kernel "
                  f"median dispatch {out['gemm']['roofline']['achieved']:.1f}",
                  file=sys.stderr, flush=True)
        if "int8" in extras:
            out["int8"] = bench_int8(ctx, lib, ops, synth, 20, 3)
            print(f"# int8 chain: {out['int8']['ms_per_chain'] * 1e3:.1f} us "
                  f"(fused, no int32 output: {out['int8']['fused']['ms_per_chain'] * 1e3:.1f} us;"
                  f" DQL {out['int8']['dql_us']:.1f} us, MatMulInteger "
                  f"{out['int8']['mmi_us']:.1f} us)", file=sys.stderr, flush=True)
        if "decode_sweep" in extras:
            sweep = []
            for m in (1, 4, 8):
                for (k, n) in synth.DECODE_PROJECTIONS:
                    r = bench_gemv(ctx, lib, ops, synth, m, k, n, 128, False, 10, 2)
                    sweep.append({kk: r[kk] for kk in ("m", "k", "n", "gbs", "sustained_us",
                                                       "dispatch_gbs", "bytes_per_call")})
            out["decode_sweep"] = sweep
            print("# decode sweep done", file=sys.stderr, flush=True)
        if "qlinear" in extras:
            out["qlinear"] = bench_qlinear(ctx, lib, ops)
            print(f"# qlinear: {json.dumps(out['qlinear'])[:300]}", file=sys.stderr, flush=True)
        if "nbits_ex" in extras:
            out["nbits_ex"] = bench_nbits_ex(ctx, lib, ops)
            print(f"# nbits_ex: {json.dumps(out['nbits_ex'])[:300]}", file=sys.stderr, flush=True)
        if "decoder" in extras:
            out["decoder"] = bench_decoder(ctx, lib)
            print(f"# decoder: decode {out['decoder']['decode_tok_s']:.0f} tok/s, prefill "
                  f"{out['decoder']['prefill_tok_s']:.0f} tok/s", file=sys.stderr, flush=True)
        if "platform" in extras:
            out["platform"] = bench_platform(ctx, lib)
            print(f"# platform: {out['platform']}", file=sys.stderr, flush=True)
    except Exception as e:  # extras must not hide the headline
        out["extras_error"] = repr(e)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(synth, args.cpu_budget if not args.quick else 6.0)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
