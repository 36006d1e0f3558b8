"""HBM-resident expert store (apus_hip_store_*) and the device-resident routed
dispatch (apus_hip_moe_routed_dev).

* Device-generated synthetic weights equal the host twin of the counter
  generator (orc_fill_bytes) byte for byte, so the oracle can rebuild them.
* apus_hip_moe_routed_dev over the store passes the per-element stage
  checks of moe_check.py on every token (w1/w3 rounding intervals, SwiGLU
  and act-quant codes, w2 and the (t, j) accumulation, pinned values exact)
  and equals the host-pointer hook bit for bit (same kernels, same data).
* store_put / store_get round-trip the six tensors of an expert.
"""
import ctypes as C
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from helpers import acts, max_rel, moe_experts, topk_routing
from moe_check import check_token

pytestmark = pytest.mark.gpu

KINDS = (0, 1, 0, 1, 0, 1)       # w1, w1s, w2, w2s, w3, w3s


def shapes(dim, inter):
    return [(inter, dim // 2), (inter, dim // 32), (dim, inter // 2), (dim, inter // 32),
            (inter, dim // 2), (inter, dim // 32)]


@pytest.fixture
def store(hip):
    made = []

    def make(L, E, dim, inter):
        err = C.create_string_buffer(256)
        st = hip.lib().apus_hip_store_create(L, E, dim, inter, err, 256)
        assert st, err.value
        made.append(st)
        return st
    yield make
    for st in made:
        hip.lib().apus_hip_store_free(st)


def read_expert(hip, st, layer, e, dim, inter):
    """The six tensors of an expert, row-major (unpacked when the store holds
    them MFMA-tiled)."""
    L = hip.lib()
    ptrs = (C.c_void_p * 6)()
    hip._check(L.apus_hip_store_get(st, layer, e, ptrs), "store_get")
    shp = shapes(dim, inter)
    srcs = list(ptrs)
    tmp = []
    if L.apus_hip_store_tiled(st):
        for m, (O, K) in enumerate(((inter, dim), (dim, inter), (inter, dim))):
            bw, bs = hip.DevBuf(int(np.prod(shp[2 * m]))), hip.DevBuf(int(np.prod(shp[2 * m + 1])))
            hip._check(L.apus_hip_unpack_weights_dev(0, srcs[2 * m], srcs[2 * m + 1], bw.ptr, bs.ptr,
                                                     O, K), "unpack")
            srcs[2 * m], srcs[2 * m + 1] = bw.ptr, bs.ptr
            tmp += [bw, bs]
        hip._check(L.apus_hip_synchronize(), "sync")
    out = []
    for p, sh in zip(srcs, shp):
        a = np.empty(sh, np.uint8)
        hip._check(L.apus_hip_d2h(a.ctypes.data, p, a.nbytes), "d2h")
        out.append(a)
    return tuple(out)


def host_expert(oracle, seed, layer, e, E, dim, inter):
    out = []
    for t, shp in enumerate(shapes(dim, inter)):
        sid = (layer * E + e) * 8 + t
        out.append(oracle.fill_bytes(seed, sid, int(np.prod(shp)), KINDS[t]).reshape(shp))
    return tuple(out)


def stage_check(hip, oracle, st, experts_of, x, idx, wgt, y, wsp, inter, tokens=None, limit=10.0):
    """Per-element checks (moe_check.check_token) of the dispatch that just
    ran on workspace wsp: the h codes and E8M0 bytes of every pair are read
    back with apus_hip_moe_routed_h."""
    L_ = hip.lib()
    s, topk = idx.shape
    hc, he = hip.DevBuf(s * topk * inter), hip.DevBuf(s * topk * (inter // 128))
    hip._check(L_.apus_hip_moe_routed_h(st, s, topk, wsp.ptr, hc.ptr, he.ptr), "routed_h")
    hcodes = hc.to_array(np.uint8, (s, topk, inter))
    he8 = he.to_array(np.uint8, (s, topk, inter // 128))
    toks = list(range(s) if tokens is None else tokens)
    # tokens in parallel (the oracle's C loops release the interpreter lock)
    with ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 4)) as ex:
        rs = list(ex.map(lambda t: check_token(oracle, experts_of, x[t], idx[t], wgt[t], limit,
                                               hcodes[t], he8[t], y[t]), toks))
    for t, r in zip(toks, rs):
        print(f"token {t}: h pinned {r['h_pinned']:.3f}, y pinned {r['y_pinned']:.3f}, "
              f"y max_rel {r['y_max_rel']:.3g}", flush=True)


def test_store_fill_matches_host_generator(hip, oracle, store):
    L, E, dim, inter = 2, 5, 512, 256
    st = store(L, E, dim, inter)
    hip._check(hip.lib().apus_hip_store_fill_random(st, 11), "fill")
    for layer, e in ((0, 0), (1, 4), (0, 3)):
        dev = read_expert(hip, st, layer, e, dim, inter)
        host = host_expert(oracle, 11, layer, e, E, dim, inter)
        for d, h in zip(dev, host):
            assert np.array_equal(d, h)


def test_store_fill_tiled_matches_host_generator(hip, oracle, store):
    """dim, inter in {2048, 4096}: the store holds MFMA-tiled matrices whose
    row-major form is the host generator's."""
    L_, E, dim, inter = 1, 3, 2048, 4096
    st = store(L_, E, dim, inter)
    assert hip.lib().apus_hip_store_tiled(st) == 1
    hip._check(hip.lib().apus_hip_store_fill_random(st, 12), "fill")
    for e in (0, 2):
        dev = read_expert(hip, st, 0, e, dim, inter)
        host = host_expert(oracle, 12, 0, e, E, dim, inter)
        for d, h in zip(dev, host):
            assert np.array_equal(d, h)


def test_store_put_get_roundtrip(hip, store, rng):
    dim, inter = 256, 128
    st = store(1, 3, dim, inter)
    ex = moe_experts(rng, 1, dim, inter)[0]
    W = [hip.ApusFp4W(t.ctypes.data_as(hip.u8p), s.ctypes.data_as(hip.u8p), o, k)
         for t, s, o, k in ((ex[0], ex[1], inter, dim), (ex[2], ex[3], dim, inter),
                            (ex[4], ex[5], inter, dim))]
    hip._check(hip.lib().apus_hip_store_put(st, 0, 2, C.byref(W[0]), C.byref(W[1]),
                                            C.byref(W[2])), "put")
    back = read_expert(hip, st, 0, 2, dim, inter)
    for a, b in zip(ex, back):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("E,dim,inter,s,topk", [(16, 512, 256, 5, 4), (32, 2048, 2048, 3, 6)])
def test_moe_routed_dev_over_store(hip, oracle, store, rng, E, dim, inter, s, topk):
    L, seed, layer = 2, 5, 1
    st = store(L, E, dim, inter)
    hip._check(hip.lib().apus_hip_store_fill_random(st, seed), "fill")
    experts = [host_expert(oracle, seed, layer, e, E, dim, inter) for e in range(E)]
    x = acts(rng, s, dim)
    idx, wgt = topk_routing(rng, s, E, topk)
    want = oracle.moe_routed(experts, x, idx, wgt, 10.0)
    L_ = hip.lib()
    dx, di, dw = (hip.DevBuf.from_array(a) for a in (x, idx, wgt))
    dy = hip.DevBuf(s * dim * 4)
    wsp = hip.DevBuf(L_.apus_hip_moe_workspace(st, s, topk))
    hip._check(L_.apus_hip_moe_routed_dev(st, layer, dx.ptr, di.ptr, dw.ptr, s, topk, 10.0,
                                          dy.ptr, wsp.ptr), "moe_routed_dev")
    got = dy.to_array(np.float32, (s, dim))
    print(f"max_rel {max_rel(got, want):.3g}")
    stage_check(hip, oracle, st, lambda e: experts[e], x, idx, wgt, got, wsp, inter)
    host = hip.moe_routed(experts, x, idx, wgt, 10.0, layer_id=777 + E)
    assert np.array_equal(got.view(np.uint32), host.view(np.uint32))


def _routed_over_store(hip, oracle, store, E, dim, inter, x, idx, wgt, seed=9):
    """Run apus_hip_moe_routed_dev over a freshly filled one-layer store and
    the oracle over host copies of the experts that the routing uses (the
    others share a placeholder: the dispatch reads only routed experts)."""
    st = store(1, E, dim, inter)
    hip._check(hip.lib().apus_hip_store_fill_random(st, seed), "fill")
    used = sorted(set(int(e) for e in idx.ravel()))
    host = {e: host_expert(oracle, seed, 0, e, E, dim, inter) for e in used}
    experts = [host.get(e, host[used[0]]) for e in range(E)]
    want = oracle.moe_routed(experts, x, idx, wgt, 10.0)
    L_ = hip.lib()
    s, topk = idx.shape
    dx, di, dw = (hip.DevBuf.from_array(a) for a in (x, idx, wgt))
    dy = hip.DevBuf(s * dim * 4)
    wsp = hip.DevBuf(L_.apus_hip_moe_workspace(st, s, topk))
    hip._check(L_.apus_hip_moe_routed_dev(st, 0, dx.ptr, di.ptr, dw.ptr, s, topk, 10.0,
                                          dy.ptr, wsp.ptr), "moe_routed_dev")
    got = dy.to_array(np.float32, (s, dim))
    print(f"max_rel {max_rel(got, want):.3g}")
    tokens = range(s) if s <= 4 else sorted(set(np.random.default_rng(s).choice(s, 4, replace=False)) | {0})
    stage_check(hip, oracle, st, lambda e: host[e], x, idx, wgt, got, wsp, inter, tokens)
    return got, want


def test_moe_routed_dev_one_token_full_shape(hip, oracle, store, rng):
    """One token at the model's shape (256 experts, dim 4096, inter 2048):
    the decode path with its compacted expert tables."""
    E, dim, inter, topk = 256, 4096, 2048, 6
    x = acts(rng, 1, dim)
    idx, wgt = topk_routing(rng, 1, E, topk)
    _routed_over_store(hip, oracle, store, E, dim, inter, x, idx, wgt)


def test_moe_routed_dev_skewed_small_batch(hip, oracle, store, rng):
    """16 tokens over 256 experts, two of them routed by most tokens: on
    average under one pair per expert, but experts 0 and 1 carry more than
    8 pairs and must take the many-row schedule."""
    E, dim, inter, s, topk = 256, 2048, 2048, 16, 6
    x = acts(rng, s, dim)
    idx = np.empty((s, topk), np.int32)
    for t in range(s):
        rest = rng.choice(np.arange(2, E), topk - 2, replace=False)
        idx[t] = np.r_[0, 1 if t < 12 else rng.integers(2, E), rest[:topk - 2]]
        while len(set(idx[t])) < topk:
            idx[t, 1] = rng.integers(2, E)
    wgt = rng.random((s, topk)).astype(np.float32)
    wgt /= wgt.sum(1, keepdims=True)
    counts = np.bincount(idx.ravel(), minlength=E)
    assert counts[0] == 16 and counts[1] >= 12 and counts.mean() < 1
    _routed_over_store(hip, oracle, store, E, dim, inter, x, idx, wgt)


def test_moe_routed_dev_duplicate_ids(hip, oracle, store, rng):
    """A token that names the same expert twice gets both pairs (each pair is
    computed and weighted on its own, as the reference's pair loop does)."""
    E, dim, inter, topk = 64, 2048, 2048, 6
    x = acts(rng, 2, dim)
    idx = np.array([[3, 3, 7, 9, 3, 11], [5, 6, 7, 8, 9, 5]], np.int32)
    wgt = rng.random((2, topk)).astype(np.float32)
    _routed_over_store(hip, oracle, store, E, dim, inter, x, idx, wgt)


def test_moe_routed_dev_graph_replays(hip, oracle, store, rng):
    """The one-token dispatch captured in a HIP graph: every replay, with
    other eager dispatches in between, equals the eager result bit for bit
    (the fused accumulation's counters are re-armed by each replay)."""
    E, dim, inter, topk, seed = 64, 4096, 2048, 6, 21
    L_ = hip.lib()
    st = store(1, E, dim, inter)
    hip._check(L_.apus_hip_store_fill_random(st, seed), "fill")
    x = acts(rng, 1, dim)
    idx, wgt = topk_routing(rng, 1, E, topk)
    idx2, wgt2 = topk_routing(rng, 1, E, topk)
    dx, di, dw, di2, dw2 = (hip.DevBuf.from_array(a) for a in (x, idx, wgt, idx2, wgt2))
    dy, dy2 = hip.DevBuf(dim * 4), hip.DevBuf(dim * 4)
    wsp = hip.DevBuf(L_.apus_hip_moe_workspace(st, 1, topk))

    def run(i, w, y):
        hip._check(L_.apus_hip_moe_routed_dev(st, 0, dx.ptr, i.ptr, w.ptr, 1, topk, 10.0,
                                              y.ptr, wsp.ptr), "moe_routed_dev")

    run(di, dw, dy)
    eager = dy.to_array(np.float32, (1, dim)).copy()
    used = sorted(set(int(e) for e in idx.ravel()))
    host = {e: host_expert(oracle, seed, 0, e, E, dim, inter) for e in used}
    stage_check(hip, oracle, st, lambda e: host[e], x, idx, wgt, eager, wsp, inter)
    run(di2, dw2, dy2)
    eager2 = dy2.to_array(np.float32, (1, dim)).copy()
    hip._check(L_.apus_hip_memset(dy.ptr, 0, dim * 4), "memset")
    hip._check(L_.apus_hip_synchronize(), "sync")
    hip._check(L_.apus_hip_graph_begin(), "graph_begin")
    run(di, dw, dy)
    hip._check(L_.apus_hip_graph_end(), "graph_end")
    for rep in range(3):
        hip._check(L_.apus_hip_memset(dy.ptr, 0, dim * 4), "memset")
        hip._check(L_.apus_hip_graph_replay(1), "replay")
        hip._check(L_.apus_hip_synchronize(), "sync")
        got = dy.to_array(np.float32, (1, dim))
        assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), rep
        run(di2, dw2, dy2)
        got2 = dy2.to_array(np.float32, (1, dim))
        assert np.array_equal(got2.view(np.uint32), eager2.view(np.uint32)), rep


@pytest.mark.parametrize("s", [1, 7])
def test_routed_with_dense_rider(hip, oracle, store, rng, s):
    """apus_hip_moe_routed_dense_dev: the routed output equals
    apus_hip_moe_routed_dev bit for bit, and the co-scheduled dense FP8
    linear [2*inter, dim] (inside the one-token w1/w3 launch at s = 1, its
    own launch in the sorted pipeline at s = 7) is within the linear bar of
    the oracle's float64 truth (one BF16 ulp + 1e-4 * esc)."""
    from helpers import bf16, bf16_linear_ok, fp8_weights
    E, dim, inter, topk = 16, 4096, 2048, 6
    st = store(1, E, dim, inter)
    L_ = hip.lib()
    hip._check(L_.apus_hip_store_fill_random(st, 3), "fill")
    x = bf16(acts(rng, s, dim))
    idx, wgt = topk_routing(rng, s, E, topk)
    w8, ws8 = fp8_weights(rng, 2 * inter, dim)
    dw, dws = hip.DevBuf(w8.nbytes), hip.DevBuf.from_array(ws8)
    raw = hip.DevBuf.from_array(w8)
    hip._check(L_.apus_hip_pack_weights_dev(1, raw.ptr, None, dw.ptr, None, 2 * inter, dim), "pack")
    dx, di, dwg = (hip.DevBuf.from_array(a) for a in (x, idx, wgt))
    y0, y1 = hip.DevBuf(s * dim * 4), hip.DevBuf(s * dim * 4)
    dout = hip.DevBuf(s * 2 * inter * 4)
    wsp = hip.DevBuf(L_.apus_hip_moe_workspace(st, s, topk))
    hip._check(L_.apus_hip_moe_routed_dev(st, 0, dx.ptr, di.ptr, dwg.ptr, s, topk, 10.0, y0.ptr,
                                          wsp.ptr), "routed_dev")
    d0 = L_.apus_hip_dispatches()
    hip._check(L_.apus_hip_moe_routed_dense_dev(st, 0, dx.ptr, di.ptr, dwg.ptr, s, topk, 10.0, y1.ptr,
                                                wsp.ptr, dw.ptr, dws.ptr, 1, dout.ptr), "routed_dense_dev")
    launches = L_.apus_hip_dispatches() - d0
    a, b = y0.to_array(np.float32, (s, dim)), y1.to_array(np.float32, (s, dim))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    got = dout.to_array(np.float32, (s, 2 * inter))
    c, sc = oracle.act_quant(x)
    truth, esc = oracle.fp8_truth(w8, ws8, c, sc)
    assert bf16_linear_ok(got, truth, 1e-4 * esc).all()
    if s == 1:
        # rider inside the w1/w3 launch; one launch in all with the one-launch layer
        assert launches == (1 if L_.apus_hip_layer1(-1, None) == 1 else 2), launches
