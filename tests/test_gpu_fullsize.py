"""Parity at the full BASELINE shapes (configs 1-4), on the GPU.

* Config 1: FP8 [4096, 4096] block-scaled GEMM at M = 512 (the tile
  schedule) against apus's own apus_fp8_gemm_mt (bitwise equal to the scalar
  normative kernel, tests/test_oracle_pin.py) on every row: max|d|/max|ref|
  <= 1e-3; err/esc <= 1e-4 on a sample of rows against the float64 truth.
* Configs 2 and 3: the routed dispatch of 64 tokens (top-6 of 256 by N(0,1)
  gating, softmax weights) and of 512 tokens (Zipf(1.1) expert popularity)
  over a 256-expert store at dim 4096, inter 2048. The reference's gate
  (tests/m9b/test_m9b.c:1-20, tests/m9e/README.md:158-164): every token's
  batched result equals dispatching that token alone, bit for bit, and so do
  the quantised SwiGLU activations h of every pair. Tokens are then checked
  stage by stage against the oracle with the per-element bounds of
  moe_check.py (whole token: h of every pair, eo and y): config 2, 8 seeded
  tokens; config 3, 8 seeded tokens, a token of the most popular expert and
  one of an expert with exactly 8 and one with exactly 9 rows (the few-row /
  many-row boundary), and in addition the h of EVERY pair routed to the
  most popular expert (so every 64-row chunk of its many-row work items,
  the last partial one included, whatever order the counting sort gave).
* Config 4: one token through a 43-layer store (147 GB resident): 6 layers
  checked stage by stage against host-regenerated experts, and the FP8
  [4096, 4096] projection of the same layers against the oracle.

The host checks run in a thread pool (the oracle's C loops release the
interpreter lock).
"""
import ctypes as C
import os
import threading
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from helpers import SUMMARY_LINES, bf16, bf16_linear_ok, err_esc, fp8_weights, max_rel
from moe_check import check_pair, check_token

pytestmark = pytest.mark.gpu

DIM, INTER, E, TOPK, LIMIT = 4096, 2048, 256, 6, 10.0
KINDS = (0, 1, 0, 1, 0, 1)       # w1, w1s, w2, w2s, w3, w3s fill kinds


def _shapes():
    return [(INTER, DIM // 2), (INTER, DIM // 32), (DIM, INTER // 2), (DIM, INTER // 32),
            (INTER, DIM // 2), (INTER, DIM // 32)]


def host_expert(oracle, seed, layer, e, n_experts=E):
    """The store's synthetic expert (layer, e), regenerated on the host by the
    same counter generator (stream id (layer * E + e) * 8 + tensor)."""
    return tuple(oracle.fill_bytes(seed, (layer * n_experts + e) * 8 + t, int(np.prod(shp)),
                                   KINDS[t]).reshape(shp)
                 for t, shp in enumerate(_shapes()))


def gate_routing(rng, s):
    logits = rng.standard_normal((s, E)).astype(np.float32)
    idx = np.argsort(-logits, axis=1, kind="stable")[:, :TOPK].astype(np.int32)
    sel = np.take_along_axis(logits, idx, 1).astype(np.float64)
    w = np.exp(sel - sel.max(1, keepdims=True))
    return idx, (w / w.sum(1, keepdims=True)).astype(np.float32)


def zipf_routing(rng, s, a=1.1):
    p = 1.0 / np.arange(1, E + 1) ** a
    p = p[rng.permutation(E)]
    p /= p.sum()
    idx = np.stack([rng.choice(E, TOPK, replace=False, p=p) for _ in range(s)]).astype(np.int32)
    w = rng.random((s, TOPK)).astype(np.float32)
    return idx, (w / w.sum(1, keepdims=True)).astype(np.float32)


class Store:
    def __init__(self, hip, layers, seed):
        err = C.create_string_buffer(256)
        self.hip, self.L = hip, hip.lib()
        self.st = self.L.apus_hip_store_create(layers, E, DIM, INTER, err, 256)
        assert self.st, err.value
        hip._check(self.L.apus_hip_store_fill_random(self.st, seed), "store fill")
        self.seed = seed

    def routed(self, layer, x, idx, wgt, read_h=False):
        """apus_hip_moe_routed_dev on device copies; returns y (and h codes,
        E8M0 bytes of every pair when read_h)."""
        hip, L = self.hip, self.L
        s, topk = idx.shape
        dx, di, dw = (hip.DevBuf.from_array(np.ascontiguousarray(a)) for a in (x, idx, wgt))
        dy = hip.DevBuf(s * DIM * 4)
        wsp = hip.DevBuf(L.apus_hip_moe_workspace(self.st, s, topk))
        hip._check(L.apus_hip_moe_routed_dev(self.st, layer, dx.ptr, di.ptr, dw.ptr, s, topk, LIMIT,
                                             dy.ptr, wsp.ptr), "moe_routed_dev")
        if not read_h:
            return dy.to_array(np.float32, (s, DIM))
        hc, he = hip.DevBuf(s * topk * INTER), hip.DevBuf(s * topk * (INTER // 128))
        hip._check(L.apus_hip_moe_routed_h(self.st, s, topk, wsp.ptr, hc.ptr, he.ptr), "routed_h")
        return (dy.to_array(np.float32, (s, DIM)), hc.to_array(np.uint8, (s, topk, INTER)),
                he.to_array(np.uint8, (s, topk, INTER // 128)))

    def close(self):
        self.L.apus_hip_store_free(self.st)


@pytest.fixture(scope="module")
def store1(hip):
    st = Store(hip, 1, 31)
    yield st
    st.close()


def _expert_cache(oracle, seed, layer):
    cache = {}
    lock = threading.Lock()

    def get(e):
        with lock:
            if e in cache:
                return cache[e]
        ex = host_expert(oracle, seed, layer, e)
        with lock:
            return cache.setdefault(e, ex)
    return get


def _pool():
    return ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 4))


def report(msg):
    """Stage-check figures: printed, and kept for the end-of-run summary
    (tests/conftest.py prints them even when the test's output is
    captured)."""
    print(msg, flush=True)
    SUMMARY_LINES.append(f"[fullsize] {msg}")


def _batched_vs_per_token(store, x, idx, wgt):
    yb, hb, eb = store.routed(0, x, idx, wgt, read_h=True)
    s = x.shape[0]
    for t in range(s):
        y1, h1, e1 = store.routed(0, x[t:t + 1], idx[t:t + 1], wgt[t:t + 1], read_h=True)
        assert np.array_equal(h1[0], hb[t]) and np.array_equal(e1[0], eb[t]), f"h of token {t}"
        assert np.array_equal(y1[0].view(np.uint32), yb[t].view(np.uint32)), f"y of token {t}"
    return yb, hb, eb


def _stage_checks(oracle, store, x, idx, wgt, yb, hb, eb, tokens, layer=0, experts=None):
    experts = experts or _expert_cache(oracle, store.seed, layer)
    tokens = [int(t) for t in tokens]
    with _pool() as ex:
        rs = list(ex.map(lambda t: check_token(oracle, experts, x[t], idx[t], wgt[t], LIMIT, hb[t],
                                               eb[t], yb[t]), tokens))
    for t, r in zip(tokens, rs):
        report(f"token {t}: experts {[int(e) for e in idx[t]]}: h pinned {r['h_pinned']:.3f}, "
               f"y pinned {r['y_pinned']:.3f} (all pinned values exact), y max_rel "
               f"{r['y_max_rel']:.3g}")
    report(f"stage-checked {len(tokens)} of {x.shape[0]} tokens")


def _bf16_x(rng, s):
    return bf16(rng.standard_normal((s, DIM)).astype(np.float32))


def test_config1_fp8_gemm_m512(hip, oracle, ref):
    rng = np.random.default_rng(101)
    M, O, K = 512, 4096, 4096
    w, ws = fp8_weights(rng, O, K)
    c, s = oracle.act_quant(bf16(rng.standard_normal((M, K)).astype(np.float32)))
    got = hip.fp8_gemm(w, ws, c, s)
    want = ref.fp8_gemm_mt(w, ws, c, s)
    mr = max_rel(got, want)
    rows = np.sort(rng.choice(M, 16, replace=False))
    truth, esc = oracle.fp8_truth(w, ws, c[rows].copy(), s[rows].copy())
    ee = err_esc(got[rows], truth, esc)
    report(f"config 1 M=512: max_rel {mr:.3g}, err/esc {ee:.3g} on rows {[int(r) for r in rows]}")
    assert mr <= 1e-3 and ee <= 1e-4


def test_config2_decode_moe(hip, oracle, store1):
    rng = np.random.default_rng(202)
    s = 64
    x = _bf16_x(rng, s)
    idx, wgt = gate_routing(rng, s)
    yb, hb, eb = _batched_vs_per_token(store1, x, idx, wgt)
    _stage_checks(oracle, store1, x, idx, wgt, yb, hb, eb, rng.choice(s, 8, replace=False))


def test_config3_prefill_moe(hip, oracle, store1):
    rng = np.random.default_rng(303)
    s = 512
    x = _bf16_x(rng, s)
    idx, wgt = zipf_routing(rng, s)
    counts = np.bincount(idx.ravel(), minlength=E)
    top = int(np.argmax(counts))
    # the most popular expert runs through the many-row schedule in several
    # 64-row chunks, the rare ones through the few-row schedule
    assert counts[top] > 128 and ((counts > 0) & (counts <= 8)).any()
    yb, hb, eb = _batched_vs_per_token(store1, x, idx, wgt)
    experts = _expert_cache(oracle, store1.seed, 0)
    # h of every pair routed to the most popular expert: its many-row work
    # items cover every 64-row chunk, the last partial one included
    pairs = np.argwhere(idx == top)
    with _pool() as ex:
        pin = list(ex.map(lambda tj: check_pair(oracle, experts(top), x[tj[0]], LIMIT,
                                                hb[tj[0], tj[1]], eb[tj[0], tj[1]]), pairs))
    report(f"expert {top}: {len(pairs)} pairs ({-(-len(pairs) // 64)} chunks of 64), h stage-checked, "
           f"pinned {np.mean(pin):.3f}")
    with_top = np.nonzero((idx == top).any(1))[0]
    tokens = [int(with_top[-1])] + [int(t) for t in rng.choice(s, 8, replace=False)]
    for n in (8, 9):                                  # the few-row / many-row boundary
        es = np.nonzero(counts == n)[0]
        if es.size:
            tokens.append(int(np.nonzero((idx == es[0]).any(1))[0][0]))
            report(f"expert {int(es[0])} has {n} rows")
        else:
            report(f"no expert with exactly {n} rows in this routing")
    rare = np.nonzero((counts[idx] <= 8).any(1))[0]
    tokens.append(int(rare[0]))
    _stage_checks(oracle, store1, x, idx, wgt, yb, hb, eb, sorted(set(tokens)), experts=experts)


@pytest.mark.timeout(600)
def test_config4_full_footprint(hip, oracle):
    """43 layers of 256 experts (147 GB of expert slabs) resident; one token
    through every layer (routed dispatch + FP8 projection per layer)."""
    layers, seed = 43, 44
    CHECKED = (0, 8, 17, 21, 33, 42)
    L = hip.lib()
    st = Store(hip, layers, seed)
    try:
        rng = np.random.default_rng(404)
        x = _bf16_x(rng, 1)
        idx, wgt = gate_routing(rng, layers)          # one routing row per layer
        O = K = DIM
        wd = hip.DevBuf(O * K * layers)
        wds = hip.DevBuf((O // 128) * (K // 128) * layers)
        hip._check(L.apus_hip_fill_random(wd.ptr, O * K * layers, seed, 1 << 40, 2), "fill fp8")
        hip._check(L.apus_hip_fill_random(wds.ptr, (O // 128) * (K // 128) * layers, seed,
                                          (1 << 40) + 1, 3), "fill fp8 scales")
        dx = hip.DevBuf.from_array(x)
        hd = hip.DevBuf(DIM * 4 * layers)
        wl = hip.DevBuf(L.apus_hip_linear_workspace(1, DIM))
        outs = {}
        for l in range(layers):
            hip._check(L.apus_hip_linear_dev(1, wd.ptr + l * O * K, wds.ptr + l * (O // 128) * (K // 128),
                                             dx.ptr, hd.ptr + l * DIM * 4, 1, K, O, wl.ptr), "fp8 linear")
            outs[l] = st.routed(l, x, idx[l:l + 1], wgt[l:l + 1], read_h=l in CHECKED)
        proj = hd.to_array(np.float32, (layers, DIM))

        def one(l):
            y, hc, he = outs[l]
            return check_token(oracle, _expert_cache(oracle, seed, l), x[0], idx[l], wgt[l], LIMIT,
                               hc[0], he[0], y[0])
        with _pool() as ex:
            rs = list(ex.map(one, CHECKED))
        for l, r in zip(CHECKED, rs):
            report(f"layer {l}: h pinned {r['h_pinned']:.3f}, y pinned {r['y_pinned']:.3f}, "
                   f"y max_rel {r['y_max_rel']:.3g}")
        for l in CHECKED:
            nsc = (O // 128) * (K // 128)
            w8 = oracle.fill_bytes(seed, 1 << 40, O * K, 2, first=l * O * K).reshape(O, K)
            s8 = oracle.fill_bytes(seed, (1 << 40) + 1, nsc, 3, first=l * nsc).reshape(O // 128, K // 128)
            c, sc = oracle.act_quant(x)
            truth, esc = oracle.fp8_truth(w8, s8, c, sc)
            assert bf16_linear_ok(proj[l:l + 1], truth, 1e-4 * esc).all(), l
    finally:
        st.close()
