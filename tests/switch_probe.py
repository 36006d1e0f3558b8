"""Child process of tests/test_gpu_switches.py: runs a fixed set of launches
with whatever APUS_HIP_* schedule switches the parent put in the environment
(they are read once per process) and writes every output to an .npz file.

Usage: python tests/switch_probe.py OUT.npz

Cases (all seeded, the same in every run):
* routed dispatch over a 16-expert store at dim 4096 / inter 2048, top-6,
  s = 1, 2, 4 (one-token and per-pair kernels) and 64 (sorted: few-row and
  many-row schedules): y and the h codes / scale bytes of every pair;
* the whole MoE sublayer at s = 8 (router, top-k, routed, FP8 shared
  expert, sum): out, routed, shared;
* dense decode-schedule launches: an FP8 [4096, 4096] GEMV at M = 1 and a
  12-entry MXFP4 [2048, 4096] grouped GEMV; dense tile-schedule launches:
  FP8 GEMMs of 100 x 512 x 4096 and 70 x 384 x 2048, and of 48, 12 and 29
  rows (the narrow schedule); split-K GEMV launches: FP8 GEMMs of 3 x 512 x
  4096 and 1 x 1024 x 8192 and a 4-row fp32 linear 512 x 4096, MXFP4 GEMMs
  of 2 x 384 x 4096 and a 4-row fp32 linear 2048 x 4096 (inputs saved for
  the oracle).
"""
import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
for p in (os.path.join(ROOT, "apus-deepseek-v4-flash_amd"), os.path.join(ROOT, "oracle"), HERE):
    sys.path.insert(0, p)

import apus_hip as hip  # noqa: E402
from helpers import acts, bf16, fp4_weights, fp8_weights, topk_routing  # noqa: E402

DIM, INTER, E, TOPK, LIMIT = 4096, 2048, 16, 6, 10.0


def routed(L, st, s, rng, out):
    x = bf16(acts(rng, s, DIM))
    idx, wgt = topk_routing(rng, s, E, TOPK)
    dx, di, dw = (hip.DevBuf.from_array(np.ascontiguousarray(a)) for a in (x, idx, wgt))
    dy = hip.DevBuf(s * DIM * 4)
    wsp = hip.DevBuf(L.apus_hip_moe_workspace(st, s, TOPK))
    hip._check(L.apus_hip_moe_routed_dev(st, 0, dx.ptr, di.ptr, dw.ptr, s, TOPK, LIMIT, dy.ptr,
                                         wsp.ptr), "routed_dev")
    hc, he = hip.DevBuf(s * TOPK * INTER), hip.DevBuf(s * TOPK * (INTER // 128))
    hip._check(L.apus_hip_moe_routed_h(st, s, TOPK, wsp.ptr, hc.ptr, he.ptr), "routed_h")
    out[f"y{s}"] = dy.to_array(np.float32, (s, DIM))
    out[f"hc{s}"] = hc.to_array(np.uint8, (s * TOPK, INTER))
    out[f"he{s}"] = he.to_array(np.uint8, (s * TOPK, INTER // 128))


def sublayer(L, st, rng, out):
    from test_gpu_moe_forward import _case, _run_device
    cfg, shared, x = _case(rng, E, DIM, INTER, 8, TOPK, False)
    o, r, sh, _, idx, _ = _run_device(hip, st, cfg, shared, bf16(x), shared_tiled=True)
    out["fwd_out"], out["fwd_routed"], out["fwd_shared"], out["fwd_idx"] = o, r, sh, idx


def dense(rng, out):
    w, ws = fp8_weights(rng, 4096, 4096)
    c, s = hip.act_quant(acts(rng, 1, 4096))
    out["fp8_w"], out["fp8_ws"], out["fp8_c"], out["fp8_s"] = w, ws, c, s
    out["fp8_y"] = hip.fp8_gemm(w, ws, c, s)
    c4, s4 = hip.act_quant(acts(rng, 1, 4096))
    ents = []
    for i in range(12):
        w4, ws4 = fp4_weights(rng, 2048, 4096)
        ents.append((w4, ws4, 0, 1))
        out[f"fp4_w{i}"], out[f"fp4_ws{i}"] = w4, ws4
    out["fp4_c"], out["fp4_s"] = c4, s4
    # dense FP8 GEMMs with more than 8 rows (the tile schedules; weights kept
    # MFMA-tiled by the dense cache)
    for name, (M, O, K) in (("t1", (100, 512, 4096)), ("t2", (70, 384, 2048)), ("t3", (48, 512, 4096)),
                            ("t4", (12, 256, 2048)), ("t5", (29, 384, 4096))):
        w, ws = fp8_weights(rng, O, K)
        c, sc = hip.act_quant(acts(rng, M, K))
        out[f"{name}_w"], out[f"{name}_ws"], out[f"{name}_c"], out[f"{name}_s"] = w, ws, c, sc
        out[f"{name}_y"] = hip.fp8_gemm(w, ws, c, sc)
    # few-row dense FP8 on tiled weights with few output rows (the split-K
    # GEMV): codes in, and an fp32-row linear (quantised in the kernel)
    for name, (M, O, K) in (("t6", (3, 512, 4096)), ("t7", (1, 1024, 8192))):
        w, ws = fp8_weights(rng, O, K)
        c, sc = hip.act_quant(acts(rng, M, K))
        out[f"{name}_w"], out[f"{name}_ws"], out[f"{name}_c"], out[f"{name}_s"] = w, ws, c, sc
        out[f"{name}_y"] = hip.fp8_gemm(w, ws, c, sc)
    w, ws = fp8_weights(rng, 512, 4096)
    x = acts(rng, 4, 4096)
    out["l1_w"], out["l1_ws"], out["l1_x"] = w, ws, x
    out["l1_y"] = hip.fp8_linear(w, ws, x)
    # the same on MXFP4 weights: codes in (2 x 384 x 4096) and an fp32-row
    # linear (4 x 2048 x 4096)
    w, ws = fp4_weights(rng, 384, 4096)
    c, sc = hip.act_quant(acts(rng, 2, 4096))
    out["f1_w"], out["f1_ws"], out["f1_c"], out["f1_s"] = w, ws, c, sc
    out["f1_y"] = hip.fp4_gemm(w, ws, c, sc)
    w, ws = fp4_weights(rng, 2048, 4096)
    x = acts(rng, 4, 4096)
    out["l2_w"], out["l2_ws"], out["l2_x"] = w, ws, x
    out["l2_y"] = hip.fp4_linear(w, ws, x)
    for i, y in enumerate(hip.fp4_gemm_grouped(ents, c4, s4, 2048)):
        out[f"fp4_y{i}"] = y


def main():
    hip.enable()
    L = hip.lib()
    err = C.create_string_buffer(256)
    st = L.apus_hip_store_create(1, E, DIM, INTER, err, 256)
    assert st, err.value
    hip._check(L.apus_hip_store_fill_random(st, 31), "store fill")
    out = {}
    rng = np.random.default_rng(77)
    for s in (1, 2, 4, 64):
        print(f"switch_probe: routed s={s}", flush=True)
        routed(L, st, s, rng, out)
    print("switch_probe: sublayer s=8", flush=True)
    sublayer(L, st, rng, out)
    print("switch_probe: dense", flush=True)
    dense(rng, out)
    hip._check(L.apus_hip_synchronize(), "sync")
    L.apus_hip_store_free(st)
    np.savez(sys.argv[1], **out)
    print("switch_probe: done", flush=True)


if __name__ == "__main__":
    main()
