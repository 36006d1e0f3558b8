"""The whole MoE sublayer on the device (apus_hip_moe_forward_dev) against
the oracle's restatement of apus_moe_forward (c/moe.h:369-595).

The device router sums the gate dot products in another order than the CPU's
sequential loop and uses ROCm's expf/log1pf/sqrtf, so its scores agree within
fp32 rounding, not bit for bit. The bars:

* scores sp: |d| <= 1e-5 * max(1, |sp|) elementwise;
* expert ids: equal for every token whose k-th and (k+1)-th selection scores
  are more than 1e-4 apart (a closer pair may swap under rounding; such
  tokens are left out of every comparison below); hash routing: equal always;
* weights: relative 1e-5;
* routed, shared and final outputs: max |d| / max |ref| <= 2^-6 and
  mean |d| / mean |ref| <= 2^-9; at the model's shape the routed output of
  every token is also held per element, stage by stage, to the rounding
  intervals of moe_check.py, given the device's own expert ids and weights. Each expert is a chain of BF16-rounded
  linears with an E4M3 re-quantisation of h between them: a one-ulp BF16
  difference in g or u (fp32 sums in another order rounding the other way)
  can move an h element to the neighbouring E4M3 code, a 2^-3 relative step
  of that element, which reaches the output scaled by its weight column. A
  single expert (the shared one) shows that as a few outputs about two BF16
  ulps of the largest output off; the routed sum of six experts averages it.

Exact ties (identical gate rows, equal bias) must pick the lowest index, as
the CPU's strict-greater-than scan does (c/attn.h:668-686).
"""
import ctypes as C
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from helpers import acts, bf16, fp8_weights, max_rel, moe_experts

pytestmark = pytest.mark.gpu


def _pack_fp8_np(w, O, K):
    """FP8 MFMA-tiled layout: [O/16][K/128][2 halves][64 lanes][16 B]."""
    return w.reshape(O // 16, 16, K // 128, 2, 4, 16).transpose(0, 2, 3, 4, 1, 5).reshape(w.shape)


def _case(rng, E, dim, inter, s, topk, hash_, gate_scale=1.0):
    sw = [fp8_weights(rng, inter, dim), fp8_weights(rng, dim, inter), fp8_weights(rng, inter, dim)]
    cfg = {"E": E, "topk": topk, "dim": dim, "inter": inter, "route_scale": 2.5, "limit": 10.0,
           "hash": hash_,
           "gate_w": (rng.standard_normal((E, dim)) * gate_scale / np.sqrt(dim)).astype(np.float32),
           "gate_bias": (rng.standard_normal(E) * 0.05).astype(np.float32)}
    if hash_:
        cfg["tid2eid"] = np.stack([rng.choice(E, topk, replace=False)
                                   for _ in range(13)]).astype(np.int64)
        cfg["ids"] = rng.integers(0, 13, s).astype(np.int64)
    shared = (sw[0][0], sw[0][1], sw[1][0], sw[1][1], sw[2][0], sw[2][1])
    return cfg, shared, acts(rng, s, dim)


def _run_device(hip, st, cfg, shared, x, shared_tiled=False, ws_out=None):
    L = hip.lib()
    s, dim = x.shape
    E, topk, inter = cfg["E"], cfg["topk"], cfg["inter"]
    keep = []

    def dev(a):
        b = hip.DevBuf.from_array(a)
        keep.append(b)
        return b.ptr
    sw = list(shared)
    if shared_tiled:
        sw[0] = _pack_fp8_np(sw[0], inter, dim)
        sw[2] = _pack_fp8_np(sw[2], dim, inter)
        sw[4] = _pack_fp8_np(sw[4], inter, dim)
    ml = hip.ApusHipMoeLayer()
    ml.gate_w = dev(cfg["gate_w"])
    ml.gate_bias = dev(cfg["gate_bias"]) if cfg.get("gate_bias") is not None else None
    ml.tid2eid = dev(cfg["tid2eid"]) if cfg["hash"] else None
    ml.hash = int(cfg["hash"])
    ml.route_scale, ml.limit = cfg["route_scale"], cfg["limit"]
    ml.sw1, ml.sw1s, ml.sw2, ml.sw2s, ml.sw3, ml.sw3s = (dev(a) for a in sw)
    ml.shared_tiled = int(shared_tiled)
    dx = dev(x)
    dids = dev(cfg["ids"]) if cfg["hash"] else None
    outs = {n: hip.DevBuf(max(1, int(np.prod(sh))) * 4) for n, sh in (
        ("out", (s, dim)), ("sp", (s, E)), ("idx", (s, topk)), ("wgt", (s, topk)),
        ("routed", (s, dim)), ("shared", (s, dim)))}
    im = hip.ApusHipMoeInterm(outs["sp"].ptr, outs["idx"].ptr, outs["wgt"].ptr,
                              outs["routed"].ptr, outs["shared"].ptr)
    wsp = hip.DevBuf(L.apus_hip_moe_forward_workspace(st, s, topk))
    hip._check(L.apus_hip_moe_forward_dev(st, 0, C.byref(ml), dx, dids, s, topk, outs["out"].ptr,
                                          C.byref(im), wsp.ptr), "moe_forward_dev")
    hip._check(L.apus_hip_synchronize(), "sync")
    if ws_out is not None:
        ws_out.append(wsp)      # the routed dispatch's workspace is its first part
    f = lambda n, sh, dt=np.float32: outs[n].to_array(dt, sh)  # noqa: E731
    return (f("out", (s, dim)), f("routed", (s, dim)), f("shared", (s, dim)), f("sp", (s, E)),
            f("idx", (s, topk), np.int32), f("wgt", (s, topk)))


def _put_experts(hip, st, experts, dim, inter):
    for e, ex in enumerate(experts):
        W = [hip.ApusFp4W(t.ctypes.data_as(hip.u8p), sc.ctypes.data_as(hip.u8p), o, k)
             for t, sc, o, k in ((ex[0], ex[1], inter, dim), (ex[2], ex[3], dim, inter),
                                 (ex[4], ex[5], inter, dim))]
        hip._check(hip.lib().apus_hip_store_put(st, 0, e, C.byref(W[0]), C.byref(W[1]),
                                                C.byref(W[2])), "put")


@pytest.fixture
def store1(hip):
    made = []

    def make(E, dim, inter):
        err = C.create_string_buffer(256)
        st = hip.lib().apus_hip_store_create(1, E, dim, inter, err, 256)
        assert st, err.value
        made.append(st)
        return st
    yield make
    for st in made:
        hip.lib().apus_hip_store_free(st)


def _clear_tokens(cfg, sp_ref):
    """Tokens whose k-th and (k+1)-th selection scores differ by more than 1e-4."""
    if cfg["hash"]:
        return np.ones(sp_ref.shape[0], bool)
    sel = np.sort(sp_ref.astype(np.float64) + cfg["gate_bias"], axis=1)[:, ::-1]
    k = cfg["topk"]
    if k >= sel.shape[1]:
        return np.ones(sp_ref.shape[0], bool)
    return (sel[:, k - 1] - sel[:, k]) > 1e-4


def mean_rel(got, want):
    want = np.asarray(want, np.float64)
    return float(np.abs(np.asarray(got, np.float64) - want).mean() / np.abs(want).mean())


def _compare(got, want, cfg):
    out, routed, shared, sp, idx, wgt = got
    w_out, w_routed, w_shared, w_sp, w_idx, w_wgt = want
    assert np.all(np.abs(sp.astype(np.float64) - w_sp) <= 1e-5 * np.maximum(1.0, np.abs(w_sp)))
    ok = _clear_tokens(cfg, w_sp)
    assert ok.sum() >= max(1, len(ok) // 2), "too few tokens without near-ties"
    assert np.array_equal(idx[ok], w_idx[ok])
    assert max_rel(wgt[ok], w_wgt[ok]) <= 1e-5
    for a, b in ((shared, w_shared), (routed[ok], w_routed[ok]), (out[ok], w_out[ok])):
        assert max_rel(a, b) <= 2.0 ** -6
        assert mean_rel(a, b) <= 2.0 ** -9
    # the final sum, fused into the routed path's last launch, is exactly
    # bf16(routed + shared) (c/moe.h:588-589)
    assert np.array_equal(out.view(np.uint32), bf16(routed + shared).view(np.uint32))


@pytest.mark.parametrize("s,topk,hash_,gate_scale", [(1, 4, 0, 1.0), (7, 4, 0, 1.0), (5, 4, 1, 1.0),
                                                      (4, 6, 0, 40.0)])
def test_moe_forward_dev_small(hip, oracle, store1, rng, s, topk, hash_, gate_scale):
    """Small shape; gate_scale 40 puts gate dot products past 20, where the
    reference's softplus returns its argument."""
    E, dim, inter = 16, 256, 128
    experts = moe_experts(rng, E, dim, inter)
    cfg, shared, x = _case(rng, E, dim, inter, s, topk, hash_, gate_scale)
    st = store1(E, dim, inter)
    _put_experts(hip, st, experts, dim, inter)
    want = oracle.moe_forward(cfg, experts, shared, x)
    got = _run_device(hip, st, cfg, shared, x)
    _compare(got, want, cfg)


@pytest.mark.parametrize("gate_scale", [1.0, 40.0])
def test_router_many_tokens_bitwise(hip, oracle, store1, rng, gate_scale):
    """More than 8 tokens take the router kernel over (8 experts, 8 tokens)
    tiles; its scores equal, bit for bit, those of the one-expert kernel that
    calls of at most 8 tokens use (same K order, same shuffle tree), and the
    sublayer holds the oracle's bars."""
    E, dim, inter, s, topk = 16, 1024, 128, 20, 4
    experts = moe_experts(rng, E, dim, inter)
    cfg, shared, x = _case(rng, E, dim, inter, s, topk, 0, gate_scale)
    st = store1(E, dim, inter)
    _put_experts(hip, st, experts, dim, inter)
    got = _run_device(hip, st, cfg, shared, x)
    _compare(got, oracle.moe_forward(cfg, experts, shared, x), cfg)
    for a, b in ((0, 8), (8, 16), (16, 20)):
        part = _run_device(hip, st, cfg, shared, x[a:b])
        assert np.array_equal(part[3].view(np.uint32), got[3][a:b].view(np.uint32)), (a, b)


def test_moe_forward_dev_exact_ties_pick_lowest_index(hip, oracle, store1, rng):
    """All gate rows equal and no bias: every score ties, so the choice is
    experts 0..topk-1 in order, with equal weights route_scale / topk."""
    E, dim, inter, s, topk = 16, 256, 128, 3, 4
    experts = moe_experts(rng, E, dim, inter)
    cfg, shared, x = _case(rng, E, dim, inter, s, topk, 0)
    cfg["gate_w"] = np.repeat(cfg["gate_w"][:1], E, axis=0)
    cfg["gate_bias"] = np.zeros(E, np.float32)
    st = store1(E, dim, inter)
    _put_experts(hip, st, experts, dim, inter)
    want = oracle.moe_forward(cfg, experts, shared, x)
    got = _run_device(hip, st, cfg, shared, x)
    assert np.array_equal(want[4], np.tile(np.arange(topk, dtype=np.int32), (s, 1)))
    assert np.array_equal(got[4], want[4])
    assert max_rel(got[5], want[5]) <= 1e-6
    assert max_rel(got[0], want[0]) <= 2.0 ** -7


@pytest.mark.parametrize("hash_,shared_tiled,s,topk", [(0, True, 2, 6), (1, False, 1, 6),
                                                      (0, True, 4, 6), (0, True, 12, 6),
                                                      (0, False, 3, 4)])
def test_moe_forward_dev_model_shape(hip, oracle, store1, rng, hash_, shared_tiled, s, topk):
    """Decode tokens at the model's shape (256 experts, dim 4096, inter 2048),
    the store filled on the device; host copies of only the experts the
    routing picks (the rest share a placeholder, which the dispatch never
    reads). The cases cover each routed mode's fused final sum (per-pair
    kernels for top-6, with 32-column w1/w3 workgroups for 1-2 tokens and
    128-column ones, which quantise h themselves, for 4; the sorted pipeline
    for 72 pairs; the ticket path for top-4) and both shared-expert paths (up
    to 8 tokens: two fused launches; more: quantise, GEMMs, SwiGLU)."""
    from test_gpu_store import host_expert
    E, dim, inter, seed = 256, 4096, 2048, 3
    cfg, shared, x = _case(rng, E, dim, inter, s, topk, hash_)
    st = store1(E, dim, inter)
    hip._check(hip.lib().apus_hip_store_fill_random(st, seed), "fill")
    first = host_expert(oracle, seed, 0, 0, E, dim, inter)
    probe = oracle.moe_forward(cfg, [first] * E, shared, x)
    used = sorted(set(int(e) for e in probe[4].ravel()))
    with ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 4)) as ex:
        host = dict(zip(used, ex.map(lambda e: host_expert(oracle, seed, 0, e, E, dim, inter), used)))
    experts = [host.get(e, first) for e in range(E)]
    want = oracle.moe_forward(cfg, experts, shared, x)
    ws = []
    got = _run_device(hip, st, cfg, shared, x, shared_tiled, ws)
    _compare(got, want, cfg)
    # the routed output of every token, near-ties included, per element and
    # stage by stage against the device's own choice of experts and weights
    # (the bounds of moe_check.py instead of the 2^-6 output bar)
    from test_gpu_store import stage_check
    for e in set(int(v) for v in got[4].ravel()) - set(host):
        host[e] = host_expert(oracle, seed, 0, e, E, dim, inter)
    stage_check(hip, oracle, st, lambda e: host[e], x, got[4], got[5], got[1], ws[0], inter,
                limit=cfg["limit"])


def test_moe_forward_dev_graph_replays(hip, oracle, store1, rng):
    """The sublayer captured into a HIP graph (the shared expert forks onto
    its own stream and joins back inside the capture): each of three
    replays, with eager launches between them, equals the eager result."""
    E, dim, inter, s, topk, seed = 256, 4096, 2048, 1, 6, 4
    cfg, shared, x = _case(rng, E, dim, inter, s, topk, 0)
    st = store1(E, dim, inter)
    L = hip.lib()
    hip._check(L.apus_hip_store_fill_random(st, seed), "fill")
    keep = []

    def dev(a):
        b = hip.DevBuf.from_array(a)
        keep.append(b)
        return b.ptr
    ml = hip.ApusHipMoeLayer()
    ml.gate_w, ml.gate_bias, ml.hash = dev(cfg["gate_w"]), dev(cfg["gate_bias"]), 0
    ml.route_scale, ml.limit = cfg["route_scale"], cfg["limit"]
    ml.sw1, ml.sw1s, ml.sw2, ml.sw2s, ml.sw3, ml.sw3s = (dev(a) for a in shared)
    dx = dev(x)
    out = hip.DevBuf(s * dim * 4)
    wsp = hip.DevBuf(L.apus_hip_moe_forward_workspace(st, s, topk))

    def run():
        hip._check(L.apus_hip_moe_forward_dev(st, 0, C.byref(ml), dx, None, s, topk, out.ptr,
                                              None, wsp.ptr), "moe_forward_dev")
    run()
    hip._check(L.apus_hip_synchronize(), "sync")
    eager = out.to_array(np.float32, (s, dim)).copy()
    hip._check(L.apus_hip_graph_begin(), "graph_begin")
    run()
    hip._check(L.apus_hip_graph_end(), "graph_end")
    for _ in range(3):
        hip._check(L.apus_hip_memset(out.ptr, 0, s * dim * 4), "memset")
        hip._check(L.apus_hip_graph_replay(1), "replay")
        hip._check(L.apus_hip_synchronize(), "sync")
        got = out.to_array(np.float32, (s, dim))
        assert np.array_equal(got.view(np.uint32), eager.view(np.uint32))
        run()                                   # eager work between replays
        hip._check(L.apus_hip_synchronize(), "sync")
