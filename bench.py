#!/usr/bin/env python3
"""bench.py — throughput of apus's quantized-matmul hot path on one MI355X.

Headline (BASELINE.json metric "MXFP4 expert GEMV GB/s (%HBM peak) @M=1; MoE
grouped-GEMM TFLOP/s @512 tok"):
  value  = config 0: batch-1 MXFP4 expert GEMV, W [2048, 4096] (E2M1 + E8M0 per 32),
           E4M3 activations quantised per 128 as apus does. One step = one grouped
           launch of 12 GEMVs (the gate+up GEMVs of one token's 6 routed experts, as
           the decode MoE issues them), each GEMV on its own HBM-resident weight copy
           (no copy read twice in a run, so the 256 MB Infinity Cache cannot serve
           them).
           Exactly --steps launches are timed with HIP events on the backend
           stream; the stream is held on the device while the host queues the
           warm-up and the timed launches, so the interval is device time of the
           timed launches only. Single-GEMV-per-launch rates are in extras.
  extras = the other BASELINE configs (FP8 GEMV/GEMM, 64-token decode MoE,
           512-token prefill MoE grouped GEMM with TFLOP/s vs the FP4/FP8 MFMA peaks).
  cpu_baseline = apus's own CPU kernel (apus_fp4_gemm_mt, AVX2 + pthread pool,
           compiled from the apus sources into oracle/_ref) on the same config-0
           GEMV, on this host's cores, timed over a bounded sample.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-extras] [--no-cpu]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "apus-deepseek-v4-flash_amd"))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
FP4_PEAK_TFLOPS = 10100.0      # dense MXFP4 MFMA
FP8_PEAK_TFLOPS = 5000.0       # dense FP8 MFMA
METRIC = "MXFP4 expert GEMV GB/s (%HBM peak) @M=1; MoE grouped-GEMM TFLOP/s @512 tok"
# HBM bytes per grouped 12-GEMV launch measured with rocprofv3 FETCH_SIZE and
# WRITE_SIZE (FETCH scaled x2.0 from a 256 MiB copy calibration); command and
# counts in profiles/config0_mxfp4_gemv_m1.txt. Re-measure when the kernel changes.
CONFIG0_TRAFFIC_BYTES = 53663744


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Dev:
    """Device buffers through the backend's own allocator (no torch)."""

    def __init__(self, H):
        self.H = H
        self.bufs = []

    def alloc(self, nbytes):
        b = self.H.DevBuf(nbytes)
        self.bufs.append(b)
        return b

    def upload(self, a):
        b = self.H.DevBuf.from_array(a)
        self.bufs.append(b)
        return b

    def free(self, *bufs):
        """Release buffers early (the large weight rotations of one bench)."""
        self.H.synchronize()
        for b in bufs:
            self.bufs.remove(b)
            b.close()


def queue_delay_us(launches):
    """Device-side hold before the timed work: long enough for the host to
    queue the warm-up launches and a graph of `launches` kernels (a few us
    each) before the device reaches them."""
    return min(200000, 2000 + 40 * launches)


def timed_graph(H, launch, steps, warm=0, warm_launch=None):
    """Capture `steps` launches into one graph and time one replay between
    two HIP events on the backend stream. The stream is first held on the
    device (apus_hip_stream_delay) while the host queues `warm` untimed
    warm-up launches (eager, through warm_launch or launch), the start
    event and the replay, so the device runs them back to back: the
    interval holds the timed launches only, with the clocks already up
    from the warm-up and no host-side submission latency."""
    L = H.lib()
    H._check(L.apus_hip_graph_begin(), "graph_begin")
    for i in range(steps):
        launch(i)
    H._check(L.apus_hip_graph_end(), "graph_end")
    H.synchronize()
    H._check(L.apus_hip_stream_delay(queue_delay_us(steps + warm)), "stream_delay")
    for i in range(warm):
        (warm_launch or launch)(steps + i)
    H._check(L.apus_hip_timer_start(), "timer_start")
    H._check(L.apus_hip_graph_replay(1), "graph_replay")
    ms = L.apus_hip_timer_stop()
    if ms < 0:
        H._check(1, "timer_stop")
    return ms


def timed_held(H, launch, steps, warm=0):
    """Time `steps` eager launches between two HIP events on the backend
    stream, all queued while the stream is held on the device
    (apus_hip_stream_delay) behind `warm` untimed warm-up launches: the
    device runs warm-up and timed launches back to back, and the interval
    holds the timed launches only. (A graph replay adds a start-up cost of
    its own: at 20 steps it measured 3 % below these eager launches, at 256
    steps the same.)"""
    L = H.lib()
    H.synchronize()
    H._check(L.apus_hip_stream_delay(queue_delay_us(steps + warm)), "stream_delay")
    for i in range(warm):
        launch(steps + i)
    H._check(L.apus_hip_timer_start(), "timer_start")
    for i in range(steps):
        launch(i)
    ms = L.apus_hip_timer_stop()
    if ms < 0:
        H._check(1, "timer_stop")
    return ms


def timed_eager(H, launch, steps):
    L = H.lib()
    H.synchronize()
    H._check(L.apus_hip_timer_start(), "timer_start")
    for i in range(steps):
        launch(i)
    ms = L.apus_hip_timer_stop()
    if ms < 0:
        H._check(1, "timer_stop")
    return ms


# ------------------------------------------------------------------ config 0

def bench_fp4_gemv(H, dev, steps, warmup, O=2048, K=4096, copies=None, group=12, extras=True,
                   singles=768):
    """Config 0. A step is one grouped launch of `group` M=1 expert GEMVs
    (W [O, K] MXFP4), each on its own weight copy: the decode MoE issues
    exactly this launch per token and layer (gate+up of the token's 6 routed
    experts = 12 GEMVs). No copy is read twice in the warm-up and timed
    launches (group x (steps + warmup + 1) copies, at least 256; 14.5 GB at
    the default 256 steps), so no cache level can serve the weights: with
    a 1.1 GB rotation reused every 21 launches the same kernel measured 4-7 %
    faster, its weights partly held by the 256 MB Infinity Cache. `steps`
    launches, queued behind a device-side hold, are timed with HIP events on
    the backend stream -> `value`.
    Extras (single GEMVs, `singles` of them):
      serial  : one launch per GEMV, serialized on one stream;
      lanes   : one launch per GEMV, round-robin on 4 concurrent streams;
      eager   : one launch per GEMV without a graph;
      rowmajor: the grouped launch on row-major weights.
    `value` uses the MFMA-tiled layout the backend keeps resident."""
    import ctypes as C
    L = H.lib()
    if copies is None:
        copies = max(256, group * (steps + warmup + 1))
    wbytes, sbytes = O * K // 2, O * K // 32
    w = dev.alloc(wbytes * copies)
    ws = dev.alloc(sbytes * copies)
    H._check(L.apus_hip_fill_random(w.ptr, wbytes * copies, 0, 1, 0), "fill w")
    H._check(L.apus_hip_fill_random(ws.ptr, sbytes * copies, 0, 2, 1), "fill ws")
    x = np.random.default_rng(0).standard_normal((1, K)).astype(np.float32)
    dx = dev.upload(x)
    codes = dev.alloc(K)
    scales = dev.alloc(K // 128 * 4)
    H._check(L.apus_hip_act_quant_dev(dx.ptr, 1, K, codes.ptr, scales.ptr), "act_quant")
    out = dev.alloc(O * 4 * copies)
    ws_lin = dev.alloc(L.apus_hip_linear_workspace(1, K))
    # entry table: one entry per weight copy, in rotation order
    ents = (H.ApusHipGemmEnt * copies)()
    for c in range(copies):
        ents[c] = H.ApusHipGemmEnt(w.ptr + c * wbytes, ws.ptr + c * sbytes, out.ptr + c * O * 4,
                                   None, None, 0, 0, 1, 0)
    dents = dev.alloc(C.sizeof(ents))
    H._check(L.apus_hip_h2d(dents.ptr, C.addressof(ents), C.sizeof(ents)), "h2d ents")
    esz = C.sizeof(H.ApusHipGemmEnt)
    # the same copies in the MFMA-tiled resident layout
    tw = dev.alloc(wbytes * copies)
    tws = dev.alloc(sbytes * copies)
    for c in range(copies):
        H._check(L.apus_hip_pack_weights_dev(0, w.ptr + c * wbytes, ws.ptr + c * sbytes,
                                             tw.ptr + c * wbytes, tws.ptr + c * sbytes, O, K), "pack")
    tents = (H.ApusHipGemmEnt * copies)()
    for c in range(copies):
        tents[c] = H.ApusHipGemmEnt(tw.ptr + c * wbytes, tws.ptr + c * sbytes, out.ptr + c * O * 4,
                                    None, None, 0, 0, 1, 0)
    dtents = dev.alloc(C.sizeof(tents))
    H._check(L.apus_hip_h2d(dtents.ptr, C.addressof(tents), C.sizeof(tents)), "h2d tents")

    def gemv(i):
        c = i % copies
        H._check(L.apus_hip_fp4_gemm_dev(w.ptr + c * wbytes, ws.ptr + c * sbytes, codes.ptr,
                                         scales.ptr, out.ptr + c * O * 4, 1, O, K, 0), "gemv")

    def grouped(j):
        c0 = (j * group) % (copies - copies % group)
        H._check(L.apus_hip_gemm_grouped_dev(0, dents.ptr + c0 * esz, group, codes.ptr, scales.ptr,
                                             O, K, O, 0, 1), "grouped gemv")

    def grouped_tiled(j):
        c0 = (j * group) % (copies - copies % group)
        H._check(L.apus_hip_gemm_grouped_dev(0 | H.W_TILED, dtents.ptr + c0 * esz, group, codes.ptr,
                                             scales.ptr, O, K, O, 0, 1), "grouped gemv tiled")

    def linear(i):
        c = i % copies
        H._check(L.apus_hip_fp4_linear_dev(w.ptr + c * wbytes, ws.ptr + c * sbytes, dx.ptr,
                                           out.ptr + c * O * 4, 1, K, O, ws_lin.ptr), "linear")

    # first launches of the kernels (code object set-up), untimed, on the one
    # spare window of copies that the timed and warm-up launches do not use
    spare = steps + warmup
    grouped_tiled(spare)
    if extras:
        for i in range(warmup):
            gemv(spare * group + i % group)
            grouped(spare)
    H.synchronize()
    launches = steps
    # the warm-up steps run right before the timed launches (same launch,
    # further weight copies), after the device-side hold
    ms_tiled = timed_held(H, grouped_tiled, launches, warm=warmup)
    gemv_bytes = wbytes + sbytes + K + (K // 128) * 4 + O * 4
    gsteps = launches * group
    res = {"steps_timed": launches, "gemvs_timed": gsteps, "group": group, "launches": launches,
           "bytes": gemv_bytes, "launch_bytes": gemv_bytes * group, "flops": 2 * O * K,
           "tiled_gbs": gemv_bytes * gsteps / (ms_tiled * 1e-3) / 1e9,
           "tiled_launch_us": ms_tiled / launches * 1e3,
           "tiled_ms_per_step": ms_tiled / launches}
    if not extras:
        dev.free(w, ws, tw, tws)
        return res
    ms_group = timed_graph(H, grouped, launches)
    steps = singles
    ms_serial = timed_graph(H, gemv, steps)
    ms_eager = timed_eager(H, gemv, steps)
    ms_lin = timed_graph(H, linear, steps)
    LANES = 4
    H._check(L.apus_hip_lanes(LANES), "lanes")

    def gemv_lanes(i):
        if i == 0:
            H._check(L.apus_hip_fork(), "fork")
        H._check(L.apus_hip_lane(i % LANES), "lane")
        gemv(i)
        if i == steps - 1:
            H._check(L.apus_hip_join(), "join")

    ms_lanes = timed_graph(H, gemv_lanes, steps)
    # algorithmic bytes of one GEMV: weights + group scales + E4M3 codes + fp32
    # act scales + fp32 outputs; the linear reads x in fp32 instead of codes
    lin_bytes = wbytes + sbytes + K * 4 + O * 4
    res.update({
        "ms_total": ms_group,
        "gbs": gemv_bytes * gsteps / (ms_group * 1e-3) / 1e9,
        "launch_us": ms_group / launches * 1e3,
        "serial_us": ms_serial / steps * 1e3,
        "serial_gbs": gemv_bytes * steps / (ms_serial * 1e-3) / 1e9,
        "lanes_gbs": gemv_bytes * steps / (ms_lanes * 1e-3) / 1e9,
        "eager_gbs": gemv_bytes * steps / (ms_eager * 1e-3) / 1e9,
        "linear_gbs": lin_bytes * steps / (ms_lin * 1e-3) / 1e9,
        "linear_us": ms_lin / steps * 1e3,
    })
    dev.free(w, ws, tw, tws)
    return res


# ------------------------------------------------------------------ config 1

def bench_fp8(H, dev, steps, O=4096, K=4096):
    """Config 1: FP8 [4096, 4096] GEMV (M = 1) and GEMM (M = 512), and the
    same projection at batched-decode sizes M = 16, 64, on
    MFMA-tiled weights; every timed and warm-up launch reads its own weight
    copy (steps + 4 copies, 4.4 GB at 256 steps), so each launch streams its
    16.8 MB from HBM."""
    L = H.lib()
    copies = steps + 4
    wbytes, sbytes = O * K, (O // 128) * (K // 128)
    w = dev.alloc(wbytes * copies)
    ws = dev.alloc(sbytes * copies)
    H._check(L.apus_hip_fill_random(w.ptr, wbytes * copies, 1, 1, 2), "fill w8")
    H._check(L.apus_hip_fill_random(ws.ptr, sbytes * copies, 1, 2, 3), "fill ws8")
    # resident layout: MFMA-tiled (FP8 tile scales keep their layout)
    tw = dev.alloc(wbytes * copies)
    for c in range(copies):
        H._check(L.apus_hip_pack_weights_dev(1, w.ptr + c * wbytes, None, tw.ptr + c * wbytes, None,
                                             O, K), "pack w8")
    dev.free(w)
    w = tw
    res = {}
    for M in (1, 16, 64, 512):
        x = np.random.default_rng(1).standard_normal((M, K)).astype(np.float32)
        dx = dev.upload(x)
        codes, scales = dev.alloc(M * K), dev.alloc(M * K // 128 * 4)
        H._check(L.apus_hip_act_quant_dev(dx.ptr, M, K, codes.ptr, scales.ptr), "act_quant")
        out = dev.alloc(M * O * 4 * 2)

        def gemm(i, M=M, codes=codes, scales=scales, out=out):
            c = i % copies
            H._check(L.apus_hip_fp8_gemm_dev(w.ptr + c * wbytes, ws.ptr + c * sbytes, codes.ptr,
                                             scales.ptr, out.ptr + (i % 2) * M * O * 4, M, O, K,
                                             H.W_TILED), "fp8 gemm")

        n = steps if M == 1 else max(10, steps // (4 if M <= 64 else 10))
        # eager launches queued behind a device-side hold, as the headline
        # (a graph replay of these GEMMs measured slower than the launches
        # themselves); warm-up on copies the timed launches do not read
        ms = timed_held(H, gemm, n, warm=3)
        nbytes = wbytes + sbytes + M * K + M * (K // 128) * 4 + M * O * 4
        t = ms * 1e-3 / n
        res[f"M{M}"] = {"us": t * 1e6, "gbs": nbytes / t / 1e9,
                        "tflops": 2 * M * O * K / t / 1e12}
    dev.free(w, ws)
    return res


# ------------------------------------------------------------------ MoE (configs 2, 3)

# the model's dense FP8 projections (reference/config.json: dim 4096, q_lora
# 1024, 64 heads x 512, o_lora 1024 x 8 groups; the indexer's query
# projection 64 index heads x 128, c/attn.h:1116); name -> (O, K)
ATTN_FP8 = {"wq_a": (1024, 4096), "wq_b": (32768, 1024), "wkv": (512, 4096), "wo_b": (4096, 8192),
            "idx_wq_b": (8192, 1024)}


def bench_attn_fp8(H, dev, steps=64, M=1, tiled=True):
    """One-token FP8 linears at the attention shapes (fp32 x -> BF16 out, act
    quant fused), MFMA-tiled weights; every timed and warm-up launch reads
    its own weight copy (steps + 4 copies), so each launch streams from HBM
    (with 8 copies in rotation the small shapes, 32 MB and less, would sit
    in the 256 MB Infinity Cache)."""
    L = H.lib()
    out = {}
    copies = steps + 4
    for name, (O, K) in ATTN_FP8.items():
        wb, sb = O * K, (O // 128) * (K // 128)
        w = dev.alloc(wb * copies)
        ws = dev.alloc(sb * copies)
        H._check(L.apus_hip_fill_random(w.ptr, wb * copies, 3, 1, 2), "fill")
        H._check(L.apus_hip_fill_random(ws.ptr, sb * copies, 3, 2, 3), "fill")
        x = dev.upload(np.random.default_rng(1).standard_normal((M, K)).astype(np.float32))
        y = dev.alloc(M * O * 4)
        wl = dev.alloc(L.apus_hip_linear_workspace(M, K))

        def step(i, O=O, K=K, w=w, ws=ws, x=x, y=y, wl=wl, wb=wb, sb=sb):
            c = i % copies
            H._check(L.apus_hip_linear_dev(1 | (H.W_TILED if tiled else 0), w.ptr + c * wb,
                                           ws.ptr + c * sb, x.ptr, y.ptr, M, K, O, wl.ptr), "linear")

        for i in range(4):
            step(steps + i)
        H.synchronize()
        us = timed_graph(H, step, steps) * 1e3 / steps
        out[name] = {"us": us, "GBs": (wb + sb) / us / 1e3}
        dev.free(w, ws)
    return out


def bench_head(H, dev, steps=16, O=129280, K=4096):
    """LM-head GEMV (reference/config.json vocab 129280 x dim 4096, BF16
    weights, 1.06 GB), one token, FP32 accumulate, through
    apus_hip_wlinear_dev; every timed launch reads its own copy of the head
    (steps + 1 copies, 18 GB at 16 steps), so the Infinity Cache holds none
    of it."""
    L = H.lib()
    wb = O * K * 2
    copies = steps + 1
    w = dev.alloc(wb * copies)
    H._check(L.apus_hip_fill_random(w.ptr, wb * copies, 5, 7, 1), "fill")   # finite BF16 patterns
    x = dev.upload(np.random.default_rng(2).standard_normal((1, K)).astype(np.float32))
    y = dev.alloc(O * 4)

    def step(i):
        H._check(L.apus_hip_wlinear_dev(w.ptr + (i % copies) * wb, x.ptr, y.ptr, 1, K, O, 4), "head")

    step(steps)
    H.synchronize()
    us = timed_graph(H, step, steps) * 1e3 / steps
    dev.free(w)
    return {"us": us, "GBs": wb / us / 1e3}


def zipf_routing(rng, s, E, topk, a):
    """top-k distinct experts per token with popularity ~ rank^-a (random rank order)."""
    p = 1.0 / np.arange(1, E + 1) ** a
    p = p[rng.permutation(E)]
    p /= p.sum()
    idx = np.stack([rng.choice(E, topk, replace=False, p=p) for _ in range(s)]).astype(np.int32)
    w = rng.random((s, topk)).astype(np.float32)
    return idx, (w / w.sum(1, keepdims=True)).astype(np.float32)


def gate_routing(rng, s, E, topk):
    logits = rng.standard_normal((s, E)).astype(np.float32)
    idx = np.argsort(-logits, axis=1, kind="stable")[:, :topk].astype(np.int32)
    sel = np.take_along_axis(logits, idx, 1).astype(np.float64)
    w = np.exp(sel - sel.max(1, keepdims=True))
    return idx, (w / w.sum(1, keepdims=True)).astype(np.float32)


def bench_moe(H, dev, store, layers, s, idx, wgt, steps, dim=4096, inter=2048, E=256):
    L = H.lib()
    topk = idx.shape[1]
    x = np.random.default_rng(2).standard_normal((s, dim)).astype(np.float32)
    from_bf16 = (x.view(np.uint32) & 0xFFFF0000).view(np.float32)   # hidden states are BF16
    dx = dev.upload(from_bf16)
    didx, dwgt = dev.upload(idx), dev.upload(wgt)
    y = dev.alloc(s * dim * 4)
    wsp = dev.alloc(L.apus_hip_moe_workspace(store, s, topk))

    def step(i):
        H._check(L.apus_hip_moe_routed_dev(store, i % layers, dx.ptr, didx.ptr, dwgt.ptr, s, topk,
                                           10.0, y.ptr, wsp.ptr), "moe")

    for i in range(2):
        step(i)
    H.synchronize()
    ms = timed_graph(H, step, steps)
    t = ms * 1e-3 / steps
    uniq = len(np.unique(idx))
    expert_bytes = 3 * (inter * dim // 2 + inter * dim // 32)
    flops = s * topk * 2 * (3 * inter * dim)
    return {"us": t * 1e6, "tok_s": s / t, "unique_experts": uniq,
            "gbs": uniq * expert_bytes / t / 1e9, "tflops": flops / t / 1e12,
            "frac_fp4_peak": flops / t / 1e12 / FP4_PEAK_TFLOPS,
            "frac_fp8_peak": flops / t / 1e12 / FP8_PEAK_TFLOPS,
            "frac_hbm": uniq * expert_bytes / t / 1e9 / HBM_PEAK_GBS}


def bench_moe_sublayer(H, dev, store, layers, s, steps, dim=4096, inter=2048, E=256, topk=6):
    """The whole MoE sublayer on the device (apus_hip_moe_forward_dev): router
    over a random fp32 gate [E, dim] with a selection bias, routed experts from
    the store, FP8 shared expert (random bytes, read as the tiled layout), bf16
    sum. A step is one layer's sublayer for s tokens."""
    import ctypes as C
    L = H.lib()
    rng = np.random.default_rng(5)
    gate = dev.upload((rng.standard_normal((E, dim)) / np.sqrt(dim)).astype(np.float32))
    bias = dev.upload((rng.standard_normal(E) * 0.05).astype(np.float32))
    sh = []
    for O, K in ((inter, dim), (dim, inter), (inter, dim)):
        w = dev.alloc(O * K)
        H._check(L.apus_hip_fill_random(w.ptr, O * K, 21, len(sh), 2), "fill")
        scl = dev.alloc((O // 128) * (K // 128))
        H._check(L.apus_hip_fill_random(scl.ptr, (O // 128) * (K // 128), 21, 10 + len(sh), 3),
                 "fill")
        sh += [w, scl]
    ml = H.ApusHipMoeLayer()
    ml.gate_w, ml.gate_bias, ml.hash = gate.ptr, bias.ptr, 0
    ml.route_scale, ml.limit = 2.5, 10.0
    ml.sw1, ml.sw1s, ml.sw2, ml.sw2s, ml.sw3, ml.sw3s = (b.ptr for b in sh)
    ml.shared_tiled = 1
    x = rng.standard_normal((s, dim)).astype(np.float32)
    dx = dev.upload((x.view(np.uint32) & 0xFFFF0000).view(np.float32))
    out = dev.alloc(s * dim * 4)
    wsp = dev.alloc(L.apus_hip_moe_forward_workspace(store, s, topk))

    def step(i):
        H._check(L.apus_hip_moe_forward_dev(store, i % layers, C.byref(ml), dx.ptr, None, s, topk,
                                            out.ptr, None, wsp.ptr), "moe_forward")

    for i in range(2):
        step(i)
    H.synchronize()
    ms = timed_graph(H, step, steps)
    return {"us": ms * 1e3 / steps}


# ------------------------------------------------------------------ CPU baseline

def bench_full_footprint(H, dev, L=43, tokens=8, reps=3, E=256, dim=4096, inter=2048, topk=6,
                         unfused=False):
    """Config 4: L MoE layers resident in HBM (256 MXFP4 experts each, config-2
    shapes) plus one FP8 [4096, 4096] projection per layer, ~148 GB. A token
    step runs, per layer, the FP8 linear and the routed dispatch of the
    token's top-6 experts (seeded gating, different per layer and token).
    `tokens` distinct steps are captured in one HIP graph and replayed."""
    import ctypes as C
    L_ = H.lib()
    err = C.create_string_buffer(256)
    t0 = time.perf_counter()
    store = L_.apus_hip_store_create(L, E, dim, inter, err, 256)
    if not store:
        raise RuntimeError("store_create: " + err.value.decode())
    try:
        log(f"[bench] config 4: filling {L} layers x {E} experts "
            f"({L_.apus_hip_store_bytes(store) / 1e9:.1f} GB) on device")
        H._check(L_.apus_hip_store_fill_random(store, 44), "store fill")
        dbytes, dsb = dim * dim, (dim // 128) * (dim // 128)
        wd = dev.alloc(dbytes * L)
        wds = dev.alloc(dsb * L)
        H._check(L_.apus_hip_fill_random(wd.ptr, dbytes * L, 44, 1 << 40, 2), "fill fp8")
        H._check(L_.apus_hip_fill_random(wds.ptr, dsb * L, 44, (1 << 40) + 1, 3), "fill fp8 s")
        wdt = dev.alloc(dbytes * L)            # resident layout: MFMA-tiled
        for l in range(L):
            H._check(L_.apus_hip_pack_weights_dev(1, wd.ptr + l * dbytes, None, wdt.ptr + l * dbytes,
                                                  None, dim, dim), "pack fp8")
        H.synchronize()
        fill_s = time.perf_counter() - t0
        log(f"[bench] config 4: resident in {fill_s:.1f} s")
        rng = np.random.default_rng(4)
        idx = np.zeros((tokens, L, topk), np.int32)
        wgt = np.zeros((tokens, L, topk), np.float32)
        for t in range(tokens):
            i, w = gate_routing(rng, L, E, topk)
            idx[t], wgt[t] = i, w
        didx, dwgt = dev.upload(idx), dev.upload(wgt)
        x = (np.random.default_rng(5).standard_normal((1, dim)).astype(np.float32).view(np.uint32)
             & 0xFFFF0000).view(np.float32)
        dx = dev.upload(x)
        hd = dev.alloc(dim * 4)
        y = dev.alloc(dim * 4 * L)
        wsp = dev.alloc(L_.apus_hip_moe_workspace(store, 1, topk))
        per = topk * 4

        wlin = dev.alloc(L_.apus_hip_linear_workspace(1, dim))

        def step(t):
            # per layer: the FP8 projection of x and the routed dispatch of x;
            # the projection rides in the routed launch (1 launch a layer with
            # the one-launch layer, else 2: in the w1/w3 launch), or, with
            # unfused, is its own launch (3 a layer)
            for l in range(L):
                off = (t * L + l) * per
                if unfused:
                    H._check(L_.apus_hip_linear_dev(1 | H.W_TILED, wdt.ptr + l * dbytes, wds.ptr + l * dsb,
                                                    dx.ptr, hd.ptr, 1, dim, dim, wlin.ptr), "fp8 linear")
                    H._check(L_.apus_hip_moe_routed_dev(store, l, dx.ptr, didx.ptr + off,
                                                        dwgt.ptr + off, 1, topk, 10.0,
                                                        y.ptr + l * dim * 4, wsp.ptr), "moe")
                    continue
                H._check(L_.apus_hip_moe_routed_dense_dev(store, l, dx.ptr, didx.ptr + off,
                                                          dwgt.ptr + off, 1, topk, 10.0,
                                                          y.ptr + l * dim * 4, wsp.ptr,
                                                          wdt.ptr + l * dbytes, wds.ptr + l * dsb, 1,
                                                          hd.ptr), "moe + fp8 projection")

        def measure():
            d0 = L_.apus_hip_dispatches()
            step(0)
            launches = L_.apus_hip_dispatches() - d0
            H.synchronize()
            H._check(L_.apus_hip_graph_begin(), "graph_begin")
            for t in range(tokens):
                step(t)
            H._check(L_.apus_hip_graph_end(), "graph_end")
            H._check(L_.apus_hip_graph_replay(1), "warm replay")
            H.synchronize()
            H._check(L_.apus_hip_timer_start(), "timer")
            H._check(L_.apus_hip_graph_replay(reps), "replay")
            ms = L_.apus_hip_timer_stop()
            return ms * 1e-3 / (tokens * reps), launches

        t_tok, launches = measure()
        # the same steps with the two-launch layer (w1/w3, then w2), when the
        # one-launch layer is what ran above
        t_two = None
        if not unfused and L_.apus_hip_layer1(-1, None) == 1:
            L_.apus_hip_layer1(0, None)
            try:
                t_two, _ = measure()
            finally:
                L_.apus_hip_layer1(1, None)
        faults = C.c_uint(0)
        L_.apus_hip_layer1(-1, C.byref(faults))
        if faults.value:
            raise RuntimeError(f"config 4: {faults.value} workgroups gave up at the layer barrier")
        expert_bytes = 3 * (inter * dim // 2 + inter * dim // 32)
        tok_bytes = L * (topk * expert_bytes + dbytes + dsb)
        return {"tok_s": 1.0 / t_tok, "ms_per_token": t_tok * 1e3, "layers": L,
                "resident_GB": (L_.apus_hip_store_bytes(store) + (dbytes + dsb) * L) / 1e9,
                "bytes_per_token": tok_bytes, "gbs": tok_bytes / t_tok / 1e9,
                "launches_per_token": launches, "fill_s": fill_s,
                "two_launch_tok_s": (1.0 / t_two) if t_two else None}
    finally:
        L_.apus_hip_store_free(store)


def bench_store_load(H, experts=64, dim=4096, inter=2048, threads=8):
    """Expert slab loader: write a one-layer container of `experts` config-2
    experts to a temporary directory, then time apus_hip_store_load into an
    MFMA-tiled store (the freshly written shards are in the page cache, so
    this measures the pread + pinned-buffer + PCIe + pack pipeline, not a
    cold disk)."""
    import ctypes as C
    import shutil
    import tempfile
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import container_util as cu
    L_ = H.lib()
    rng = np.random.default_rng(9)
    d = tempfile.mkdtemp(prefix="apus_container_")
    try:
        arr = cu.expert_arrays(rng, dim, inter)   # one expert's bytes, reused
        entries = []
        for e in range(experts):
            entries += cu.expert_entries(0, e, arr)
        cu.write_container(d, {"model-00001.safetensors": entries})
        err = C.create_string_buffer(512)
        c = L_.apus_hip_container_open(d.encode(), 1, 0, experts, err, 512)
        if not c:
            raise RuntimeError(err.value.decode())
        st = L_.apus_hip_store_create(1, experts, dim, inter, err, 256)
        try:
            t0 = time.perf_counter()
            if L_.apus_hip_store_load(st, c, threads, err, 512):
                raise RuntimeError(err.value.decode())
            dt = time.perf_counter() - t0
            rec = H.ApusHipSlabRec()
            L_.apus_hip_container_slab(c, 0, 0, C.byref(rec))
            nbytes = rec.len * experts
        finally:
            L_.apus_hip_store_free(st)
            L_.apus_hip_container_close(c)
        return {"GBs": nbytes / dt / 1e9, "bytes": nbytes, "s": dt}
    finally:
        shutil.rmtree(d, ignore_errors=True)


_HOST_KEEP = []


def bench_hostptr(H, O=2048, K=4096, calls=400):
    """Config 0 through the host-pointer hook (apus_hip_fp4_linear, the
    c/attn.h:432 call site): weights in host memory (uploaded once into the
    backend's dense cache, keyed by pointer), x and out in host memory, so
    every call pays the x upload, the out download and a stream sync. This
    is the PCIe-inclusive rate of the boundary, reported beside `value`."""
    import ctypes as C
    rng = np.random.default_rng(0)
    w = rng.integers(0, 256, (O, K // 2), dtype=np.uint8)
    ws = rng.integers(118, 131, (O, K // 32), dtype=np.uint8)
    x = rng.standard_normal((1, K)).astype(np.float32)
    out = np.empty((1, O), np.float32)
    W = H.fp4_weight(w, ws)
    # the backend keys cached weights by host pointer: keep the arrays alive
    # for the whole process so no later allocation reuses their addresses
    _HOST_KEEP.extend([w, ws])
    L = H.lib()
    xp = x.ctypes.data_as(C.POINTER(C.c_float))
    op = out.ctypes.data_as(C.POINTER(C.c_float))

    def call():
        H._check(L.apus_hip_fp4_linear(C.byref(W), xp, op, 1, K, O), "fp4_linear (host)")

    for _ in range(20):
        call()
    t0 = time.perf_counter()
    for _ in range(calls):
        call()
    us = (time.perf_counter() - t0) / calls * 1e6
    nbytes = O * K // 2 + O * K // 32 + 4 * K + 4 * O
    return {"us": us, "GBs": nbytes / us / 1e3}


def cpu_threads():
    """Threads for apus's CPU pool: the host's usable CPUs (nproc: the
    process's affinity set), capped by OMP_NUM_THREADS where the host sets
    it (the GPU box's CPU share) and at 32 like the pool itself
    (c/pool.h:51,97-103)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, min(n, 32))


def cpu_baseline(O=2048, K=4096, budget_s=12.0):
    """apus's own apus_fp4_gemm_mt (AVX2 rows + pthread pool) on config 0."""
    threads = cpu_threads()
    os.environ.setdefault("APUS_THREADS", str(threads))
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle
    kind = "reference" if pyoracle.have_ref() else "port"
    rng = np.random.default_rng(0)
    w = rng.integers(0, 256, (O, K // 2), dtype=np.uint8)
    ws = rng.integers(118, 131, (O, K // 32), dtype=np.uint8)
    x = rng.standard_normal((1, K)).astype(np.float32)
    if kind == "reference":
        R = pyoracle.Reference()
        c, s = R.act_quant(x)
        fn = lambda: R.fp4_gemm_mt(w, ws, c, s)  # noqa: E731
        used = R.L.ref_pool_threads()
    else:
        Orc = pyoracle.Oracle()
        c, s = Orc.act_quant(x)
        fn = lambda: Orc.fp4_gemm(w, ws, c, s)  # noqa: E731
        used = 1
    fn()
    t0 = time.perf_counter()
    fn()
    one = max(time.perf_counter() - t0, 1e-6)
    reps = max(1, int(budget_s / 3 / one))
    best = None
    for _ in range(3):
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        dt = (time.perf_counter() - t0) / reps
        best = dt if best is None else min(best, dt)
    nbytes = O * K // 2 + O * K // 32 + K + (K // 128) * 4 + O * 4
    if kind == "reference":
        assert R.L.ref_x86_avx2_hits() > 0, "reference AVX2 rows were not taken"
    return {"value": nbytes / best / 1e9, "unit": "GB/s", "cores": int(used), "kind": kind,
            "host_cpus": os.cpu_count(),
            "sample": f"config 0 GEMV O={O} K={K} M=1 (apus_fp4_gemm_mt), best of 3 x {reps} "
                      f"reps, {best * 1e3:.3f} ms/GEMV; {int(used)} pool threads of "
                      f"{os.cpu_count()} host CPUs"}


def cpu_extras(budget_s=4.0):
    """apus's own CPU kernels on the other GEMM configs (reported beside the
    GPU extras, same host cores): config 1 FP8 M=1 and M=512
    (apus_fp8_gemm_mt) and one config-3 expert's w1 at 64 rows
    (apus_fp4_gemm_mt). Each is the best of 3 timings within ~budget_s."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle
    if not pyoracle.have_ref():
        return {}
    R = pyoracle.Reference()
    rng = np.random.default_rng(1)

    def best_of(fn):
        fn()
        t0 = time.perf_counter()
        fn()
        one = max(time.perf_counter() - t0, 1e-6)
        reps = max(1, int(budget_s / 3 / one))
        best = None
        for _ in range(3):
            t0 = time.perf_counter()
            for _ in range(reps):
                fn()
            dt = (time.perf_counter() - t0) / reps
            best = dt if best is None else min(best, dt)
        return best

    out = {}
    O = K = 4096
    w8 = rng.integers(0, 0x7e, (O, K), dtype=np.uint8)
    ws8 = rng.integers(117, 124, (O // 128, K // 128), dtype=np.uint8)
    for M in (1, 512):
        c, sc = R.act_quant(rng.standard_normal((M, K)).astype(np.float32))
        t = best_of(lambda c=c, sc=sc: R.fp8_gemm_mt(w8, ws8, c, sc))
        if M == 1:
            out["cpu_config1_fp8_M1_us"] = round(t * 1e6, 1)
            out["cpu_config1_fp8_M1_GBs"] = round((O * K + (O // 128) * (K // 128)) / t / 1e9, 2)
        else:
            out["cpu_config1_fp8_M512_us"] = round(t * 1e6, 1)
            out["cpu_config1_fp8_M512_TFLOPs"] = round(2.0 * M * O * K / t / 1e12, 4)
    O4, K4, M4 = 2048, 4096, 64
    w4 = rng.integers(0, 256, (O4, K4 // 2), dtype=np.uint8)
    ws4 = rng.integers(118, 131, (O4, K4 // 32), dtype=np.uint8)
    c, sc = R.act_quant(rng.standard_normal((M4, K4)).astype(np.float32))
    t = best_of(lambda: R.fp4_gemm_mt(w4, ws4, c, sc))
    out["cpu_config3_expert_w1_M64_us"] = round(t * 1e6, 1)
    out["cpu_config3_expert_w1_M64_TFLOPs"] = round(2.0 * M4 * O4 * K4 / t / 1e12, 4)
    out["cpu_threads"] = int(R.L.ref_pool_threads())
    out["cpu_host_cpus"] = os.cpu_count()
    return out


def cpu_moe(budget_s=20.0):
    """apus's own CPU path on the MoE configs, same host threads:
    * configs 2 and 3: the real apus_moe_forward (c/moe.h:369-595) with the
      expert ids forced through hash routing, on the config-2 routing (64
      tokens, top-6 of 256 by N(0,1) gating) and the config-3 routing (512
      tokens, Zipf(1.1)); experts at dim 4096 / inter 2048, expert id e
      reading slab e % 64 of a pool of 64 distinct random experts (856 MB,
      far above any CPU cache, so every expert is streamed from DRAM as a
      distinct one would be; a full 3.4 GB set only costs generation time).
      The timed call is the whole sublayer: router scores
      (gate [256, 4096]), the routed experts (its batched path for s > 1)
      and the FP8 shared expert (all-zero weights, full cost), so the
      routed part alone is somewhat faster;
    * config 4: one token through 43 layers, each the FP8 [4096, 4096]
      projection and the token's 6 routed experts as apus_moe_forward's
      one-token path runs them (ref_decode_layer), the 258 expert slabs drawn
      in turn from the pool (each re-read only after 10 layers, 550 MB
      later) and 43 distinct projections: the bytes one token touches in the
      150 GB model.
    """
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle
    if not pyoracle.have_ref():
        return {}
    R = pyoracle.Reference()
    E, dim, inter, topk = 256, 4096, 2048, 6
    rng = np.random.default_rng(11)
    t0 = time.perf_counter()
    pool = []
    for _ in range(64):
        pool.append((rng.integers(0, 256, (inter, dim // 2), dtype=np.uint8),
                        rng.integers(118, 131, (inter, dim // 32), dtype=np.uint8),
                        rng.integers(0, 256, (dim, inter // 2), dtype=np.uint8),
                        rng.integers(118, 131, (dim, inter // 32), dtype=np.uint8),
                        rng.integers(0, 256, (inter, dim // 2), dtype=np.uint8),
                        rng.integers(118, 131, (inter, dim // 32), dtype=np.uint8)))
    experts = [pool[e % len(pool)] for e in range(E)]
    gate = (rng.standard_normal((E, dim)) / np.sqrt(dim)).astype(np.float32)
    log(f"[bench] CPU MoE: experts generated in {time.perf_counter() - t0:.1f} s")
    out = {}
    ebytes = sum(a.nbytes for a in experts[0])
    # the GPU legs' routings (the same generator, drawn in the same order)
    rr = np.random.default_rng(3)
    routes = {"config2": gate_routing(rr, 64, E, topk)[0], "config3": zipf_routing(rr, 512, E, topk, 1.1)[0]}
    for cfg, s in (("config2", 64), ("config3", 512)):
        idx = routes[cfg]
        x = rng.standard_normal((s, dim)).astype(np.float32)
        t0 = time.perf_counter()
        R.moe_routed(experts, gate, x, idx, 2.5, 10.0)
        one = time.perf_counter() - t0
        reps = max(1, min(3, int(budget_s / 3 / one)))
        t0 = time.perf_counter()
        for _ in range(reps):
            R.moe_routed(experts, gate, x, idx, 2.5, 10.0)
        dt = (time.perf_counter() - t0) / reps
        uniq = len(np.unique(idx))
        out[f"cpu_{cfg}_sublayer_us"] = round(dt * 1e6, 1)
        out[f"cpu_{cfg}_tok_s"] = round(s / dt, 2)
        out[f"cpu_{cfg}_expert_GBs"] = round(uniq * ebytes / dt / 1e9, 2)
        if cfg == "config3":
            out["cpu_config3_routed_TFLOPs"] = round(2.0 * 3 * s * topk * dim * inter / dt / 1e12, 5)
        log(f"[bench] CPU {cfg}: {dt * 1e3:.1f} ms per sublayer ({reps} timed)")
    L = 43
    pw = [rng.integers(0, 0x7E, (dim, dim), dtype=np.uint8) for _ in range(L)]
    pws = [rng.integers(117, 124, (dim // 128, dim // 128), dtype=np.uint8) for _ in range(L)]
    x = rng.standard_normal(dim).astype(np.float32)
    wgt = np.full(topk, 1.0 / topk, np.float32)

    def token():
        for l in range(L):
            exs = [experts[(l * topk + j) % E] for j in range(topk)]
            pyoracle.ref_decode_layer(R, exs, wgt, pw[l], pws[l], x, 10.0)
    token()
    t0 = time.perf_counter()
    n = 0
    while n < 3 and (n == 0 or time.perf_counter() - t0 < budget_s / 3):
        token()
        n += 1
    dt = (time.perf_counter() - t0) / n
    per_tok = L * (topk * ebytes + dim * dim + (dim // 128) ** 2)
    out["cpu_config4_tok_s"] = round(1.0 / dt, 3)
    out["cpu_config4_ms_per_token"] = round(dt * 1e3, 1)
    out["cpu_config4_GBs"] = round(per_tok / dt / 1e9, 2)
    out["cpu_config4_layers"] = L
    log(f"[bench] CPU config 4: {dt * 1e3:.1f} ms per token ({n} timed)")
    return out


# ------------------------------------------------------------------ main

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256,
                    help="config-0 grouped launches timed (12 GEMVs each)")
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--skip-extras", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="", help="comma list: gemv,fp8,attn,decode,prefill,full,load")
    ap.add_argument("--full-layers", type=int, default=43,
                    help="config 4: resident MoE layers (43 fill ~148 GB)")
    ap.add_argument("--full-unfused", action="store_true",
                    help="config 4: the FP8 projection as its own launch (the pre-fusion schedule)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a plain 256 MiB device copy (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for "
              f"--gpus {args.gpus}); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import apus_hip as H
    H.enable()
    name, cus = H.device_info()
    log(f"device: {name} ({cus} CUs)")
    dev = Dev(H)
    only = set(filter(None, args.only.split(",")))
    want = (lambda k: not only or k in only)

    extras = {}
    g = None
    if want("gemv"):
        log(f"[bench] config 0 MXFP4 GEMV: {args.warmup} warmup, {args.steps} timed steps")
        g = bench_fp4_gemv(H, dev, args.steps, args.warmup, extras=not args.skip_extras)
        if not args.skip_extras:
            extras["config0_rowmajor_grouped_GBs"] = round(g["gbs"], 1)
            extras["config0_single_launch_serial_GBs"] = round(g["serial_gbs"], 1)
            extras["config0_single_launch_us"] = round(g["serial_us"], 3)
            extras["config0_single_launch_4lanes_GBs"] = round(g["lanes_gbs"], 1)
            extras["config0_linear_GBs"] = round(g["linear_gbs"], 1)
            extras["config0_linear_us"] = round(g["linear_us"], 3)
            extras["config0_eager_launch_GBs"] = round(g["eager_gbs"], 1)
            hp = bench_hostptr(H)
            extras["config0_hostptr_linear_us"] = round(hp["us"], 2)
            extras["config0_hostptr_linear_GBs"] = round(hp["GBs"], 1)
    if not args.skip_extras and want("fp8"):
        log("[bench] config 1 FP8 GEMV/GEMM")
        f8 = bench_fp8(H, dev, min(args.steps, 512))
        extras["config1_fp8_M1_GBs"] = round(f8["M1"]["gbs"], 1)
        extras["config1_fp8_M1_us"] = round(f8["M1"]["us"], 2)
        extras["config1_fp8_M512_TFLOPs"] = round(f8["M512"]["tflops"], 1)
        for mm in (16, 64):   # batched-decode sizes of the same projection
            extras[f"fp8_4096x4096_M{mm}_us"] = round(f8[f"M{mm}"]["us"], 2)
            extras[f"fp8_4096x4096_M{mm}_GBs"] = round(f8[f"M{mm}"]["gbs"], 1)
        extras["config1_fp8_M512_us"] = round(f8["M512"]["us"], 2)
    if not args.skip_extras and want("attn"):
        hd = bench_head(H, dev)
        extras["lm_head_bf16_us"] = round(hd["us"], 1)
        extras["lm_head_bf16_GBs"] = round(hd["GBs"], 1)
        for name, r in bench_attn_fp8(H, dev).items():
            extras[f"attn_{name}_M1_us"] = round(r["us"], 2)
            extras[f"attn_{name}_M1_GBs"] = round(r["GBs"], 1)
    if not args.skip_extras and (want("decode") or want("prefill")):
        layers = 4
        err = __import__("ctypes").create_string_buffer(256)
        store = H.lib().apus_hip_store_create(layers, 256, 4096, 2048, err, 256)
        if not store:
            raise RuntimeError(err.value.decode())
        H._check(H.lib().apus_hip_store_fill_random(store, 7), "store fill")
        rng = np.random.default_rng(3)
        if want("decode"):
            log("[bench] config 2 decode MoE, 64 tokens top-6 of 256")
            idx, wgt = gate_routing(rng, 64, 256, 6)
            d = bench_moe(H, dev, store, layers, 64, idx, wgt, min(64, args.steps))
            extras.update({"config2_decode_tok_s": round(d["tok_s"], 1),
                           "config2_decode_us": round(d["us"], 1),
                           "config2_decode_GBs": round(d["gbs"], 1),
                           "config2_unique_experts": d["unique_experts"]})
            for sl in (1, 64):
                r = bench_moe_sublayer(H, dev, store, layers, sl, min(64, args.steps))
                extras[f"moe_sublayer_s{sl}_us"] = round(r["us"], 1)
        if want("prefill"):
            log("[bench] config 3 prefill MoE, 512 tokens top-6 of 256, Zipf(1.1)")
            idx, wgt = zipf_routing(rng, 512, 256, 6, 1.1)
            p = bench_moe(H, dev, store, layers, 512, idx, wgt, min(16, args.steps))
            extras.update({"config3_prefill_TFLOPs": round(p["tflops"], 2),
                           "config3_prefill_us": round(p["us"], 1),
                           "config3_frac_fp4_peak": round(p["frac_fp4_peak"], 5),
                           "config3_frac_fp8_peak": round(p["frac_fp8_peak"], 5),
                           "config3_weight_GBs": round(p["gbs"], 1),
                           "config3_unique_experts": p["unique_experts"]})
        H.lib().apus_hip_store_free(store)
    if not args.skip_extras and want("full"):
        log("[bench] config 4 full-footprint decode")
        f = bench_full_footprint(H, dev, L=args.full_layers, unfused=args.full_unfused)
        extras.update({"config4_tok_s": round(f["tok_s"], 1),
                       "config4_ms_per_token": round(f["ms_per_token"], 3),
                       "config4_GBs": round(f["gbs"], 1),
                       "config4_hbm_frac": round(f["gbs"] / HBM_PEAK_GBS, 4),
                       "config4_layers": f["layers"],
                       "config4_resident_GB": round(f["resident_GB"], 1),
                       "config4_bytes_per_token": f["bytes_per_token"],
                       "config4_launches_per_token": f["launches_per_token"],
                       "config4_two_launch_layer_tok_s": (round(f["two_launch_tok_s"], 1)
                                                          if f["two_launch_tok_s"] else None)})

    if not args.skip_extras and want("load"):
        log("[bench] expert slab loader: 64 experts from a page-cached container")
        ld = bench_store_load(H)
        extras.update({"store_load_GBs": round(ld["GBs"], 2), "store_load_bytes": ld["bytes"]})
    if args.calibrate_copy:
        # a plain copy of known size: its FETCH_SIZE / WRITE_SIZE counters give
        # the scale between the counters and bytes moved
        nb = 256 << 20
        src, dst = dev.alloc(nb), dev.alloc(nb)
        H._check(H.lib().apus_hip_fill_random(src.ptr, nb, 9, 9, 0), "fill")
        for _ in range(2):
            H._check(H.lib().apus_hip_d2d(dst.ptr, src.ptr, nb), "d2d")
        H.synchronize()
        log(f"[bench] calibration copy: 2 x {nb} bytes")
    cpu = None if args.no_cpu else cpu_baseline()
    if cpu is not None and not args.skip_extras:
        log("[bench] CPU reference on configs 1 and 3 (samples)")
        extras.update(cpu_extras())
        extras.update(cpu_moe())
    if g is None:
        print(json.dumps({"metric": METRIC, "extras": extras, "cpu_baseline": cpu}))
        return
    line = {
        "metric": METRIC,
        "value": round(g["tiled_gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": g["steps_timed"],
        "warmup": args.warmup,
        "ms_per_step": g["tiled_ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "e4m3 x e2m1 (fp32 accumulate)",
        "data": "synthetic: weights from a counter hash on device (uniform nibbles, E8M0 "
                "118..130), x ~ N(0,1) seed 0",
        "config": {"workload": "config 0: MXFP4 expert GEMV O=2048 K=4096 M=1; one step = one "
                               f"grouped launch of {g['group']} such GEMVs (gate+up of one token's 6 "
                               "routed experts, as the decode MoE issues them), each on its own "
                               "HBM-resident weight copy (no copy read twice in the warm-up and "
                               "timed launches); weights in the MFMA-tiled layout the backend's "
                               "caches and expert store keep",
                   "group": g["group"], "gemvs_timed": g["gemvs_timed"],
                   "hbm_frac": round(g["tiled_gbs"] / HBM_PEAK_GBS, 4),
                   },
        # the dominant kernel is the grouped GEMM launch; the steps run back
        # to back (the device holds the stream until the host has queued
        # them), so per-launch time = kernel duration plus the inter-kernel
        # gap (compare rocprofv3's average)
        "roofline": {"bound": "hbm",
                     "achieved": round(g["launch_bytes"] / (g["tiled_launch_us"] * 1e-6) / 1e9, 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(g["launch_bytes"] / (g["tiled_launch_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "kernel": "apus_gemv_grp_kernel (grouped, 12 GEMVs, tiled weights)",
                     "launch_us": round(g["tiled_launch_us"], 3), "bytes_per_launch": g["launch_bytes"],
                     "traffic": CONFIG0_TRAFFIC_BYTES,
                     "traffic_source": "rocprofv3 FETCH_SIZE + WRITE_SIZE per launch, calibrated "
                                       "against a 256 MiB copy (profiles/config0_mxfp4_gemv_m1.txt); "
                                       "not measured in this run"},
        "cpu_baseline": cpu,
        "extras": extras,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
