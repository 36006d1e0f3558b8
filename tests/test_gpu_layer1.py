"""The one-launch one-token MoE layer (apus_moe_layer1_kernel) on the GPU.

It replaces the two one-token launches (w1/w3 with the h hand-off, then w2
with the accumulation) by one kernel with a grid-wide barrier between the
phases, and must give the same y bit for bit. apus_hip_layer1 switches it on
and off in one process, so every case runs both ways on the same inputs:

* routed dispatch over an expert store (dim 4096, inter 2048, 256 experts,
  top-6): y and the quantised h of every pair bit-identical, one launch
  against two; routings with a repeated expert and with an expert id out of
  range (the pair is skipped, as in the reference's bounds check);
* with the dense FP8 rider [4096, 4096]: y bit-identical, the rider's output
  (two K chains instead of one) within the linear bar of the float64 truth;
* eight layers' launches captured in one graph and replayed three times, each
  replay bit-identical to the eager results (the barrier's counter returns to
  zero after every launch);
* no workgroup gave up waiting at the barrier in any of these launches.
"""
import ctypes as C

import numpy as np
import pytest

from helpers import bf16, bf16_linear_ok, fp8_weights, topk_routing

pytestmark = pytest.mark.gpu

DIM, INTER, E, TOPK, LIMIT = 4096, 2048, 256, 6, 10.0


@pytest.fixture(scope="module")
def st8(hip):
    L = hip.lib()
    err = C.create_string_buffer(256)
    st = L.apus_hip_store_create(8, E, DIM, INTER, err, 256)
    assert st, err.value
    hip._check(L.apus_hip_store_fill_random(st, 81), "store fill")
    if L.apus_hip_layer1(-1, None) < 0:
        pytest.fail(L.apus_hip_last_error().decode())
    yield st
    L.apus_hip_layer1(1, None)
    L.apus_hip_store_free(st)


def _layer1_available(hip):
    L = hip.lib()
    on = L.apus_hip_layer1(1, None)
    assert on >= 0, L.apus_hip_last_error().decode()
    if on == 0:
        pytest.skip("the one-launch layer needs 256 resident workgroups (fewer CUs here)")


def _faults(hip):
    f = C.c_uint(0)
    assert hip.lib().apus_hip_layer1(-1, C.byref(f)) >= 0
    return f.value


def _routed(hip, st, layer, x, idx, wgt, rider=None):
    """y, h codes, h scale bytes and launch count of one routed call (with
    rider = (w, ws) device buffers: routed_dense_dev, returning its output
    too)."""
    L = hip.lib()
    s = x.shape[0]
    dx, di, dw = (hip.DevBuf.from_array(np.ascontiguousarray(a)) for a in (x, idx, wgt))
    dy = hip.DevBuf(s * DIM * 4)
    wsp = hip.DevBuf(L.apus_hip_moe_workspace(st, s, TOPK))
    d0 = L.apus_hip_dispatches()
    dout = None
    if rider is None:
        hip._check(L.apus_hip_moe_routed_dev(st, layer, dx.ptr, di.ptr, dw.ptr, s, TOPK, LIMIT,
                                             dy.ptr, wsp.ptr), "routed_dev")
    else:
        dout = hip.DevBuf(s * 2 * INTER * 4)
        hip._check(L.apus_hip_moe_routed_dense_dev(st, layer, dx.ptr, di.ptr, dw.ptr, s, TOPK, LIMIT,
                                                   dy.ptr, wsp.ptr, rider[0].ptr, rider[1].ptr, 1,
                                                   dout.ptr), "routed_dense_dev")
    launches = L.apus_hip_dispatches() - d0
    hc, he = hip.DevBuf(s * TOPK * INTER), hip.DevBuf(s * TOPK * (INTER // 128))
    hip._check(L.apus_hip_moe_routed_h(st, s, TOPK, wsp.ptr, hc.ptr, he.ptr), "routed_h")
    out = dout.to_array(np.float32, (s, 2 * INTER)) if dout is not None else None
    return (dy.to_array(np.float32, (s, DIM)), hc.to_array(np.uint8, (s, TOPK, INTER)),
            he.to_array(np.uint8, (s, TOPK, INTER // 128)), launches, out)


def _both(hip, st, layer, x, idx, wgt, rider=None):
    L = hip.lib()
    assert L.apus_hip_layer1(1, None) == 1
    one = _routed(hip, st, layer, x, idx, wgt, rider)
    assert L.apus_hip_layer1(0, None) == 0
    two = _routed(hip, st, layer, x, idx, wgt, rider)
    assert L.apus_hip_layer1(1, None) == 1
    return one, two


def _routing(rng, case):
    idx, wgt = topk_routing(rng, 1, E, TOPK)
    if case == "repeat":
        idx[0, 4] = idx[0, 1]                       # the same expert in two slots
    elif case == "out_of_range":
        idx[0, 2] = E + 3                           # skipped pair
        idx[0, 5] = -1
    return idx, wgt


@pytest.mark.parametrize("case", ["plain", "repeat", "out_of_range"])
def test_layer1_equals_two_launches(hip, st8, case):
    _layer1_available(hip)
    rng = np.random.default_rng({"plain": 1, "repeat": 2, "out_of_range": 3}[case])
    for layer in (0, 5):
        x = bf16(rng.standard_normal((1, DIM)).astype(np.float32))
        idx, wgt = _routing(rng, case)
        (y1, h1, e1, n1, _), (y2, h2, e2, n2, _) = _both(hip, st8, layer, x, idx, wgt)
        assert (n1, n2) == (1, 2), (n1, n2)
        assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32)), f"y, layer {layer}"
        ok = (idx[0] >= 0) & (idx[0] < E)
        assert np.array_equal(h1[0, ok], h2[0, ok]) and np.array_equal(e1[0, ok], e2[0, ok])
        assert np.isfinite(y1).all() and np.abs(y1).max() > 0
    assert _faults(hip) == 0


def test_layer1_with_dense_rider(hip, oracle, st8):
    _layer1_available(hip)
    L = hip.lib()
    rng = np.random.default_rng(4)
    w8, ws8 = fp8_weights(rng, 2 * INTER, DIM)
    raw = hip.DevBuf.from_array(w8)
    dwt, dws = hip.DevBuf(w8.nbytes), hip.DevBuf.from_array(ws8)
    hip._check(L.apus_hip_pack_weights_dev(1, raw.ptr, None, dwt.ptr, None, 2 * INTER, DIM), "pack")
    x = bf16(rng.standard_normal((1, DIM)).astype(np.float32))
    idx, wgt = _routing(rng, "plain")
    (y1, h1, _, n1, o1), (y2, h2, _, n2, o2) = _both(hip, st8, 3, x, idx, wgt, (dwt, dws))
    assert (n1, n2) == (1, 2), (n1, n2)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    assert np.array_equal(h1, h2)
    c, sc = oracle.act_quant(x)
    truth, esc = oracle.fp8_truth(w8, ws8, c, sc)
    assert bf16_linear_ok(o1, truth, 1e-4 * esc).all()
    assert bf16_linear_ok(o2, truth, 1e-4 * esc).all()
    print(f"rider: {int((o1 != o2).sum())} of {o1.size} outputs differ by K-chain order")
    assert _faults(hip) == 0


def test_layer1_graph_replays(hip, st8):
    """Eight layers of one token each, captured once and replayed three times
    with eager work between the replays; every replay equals the eager run."""
    _layer1_available(hip)
    L = hip.lib()
    rng = np.random.default_rng(5)
    layers = 8
    x = bf16(rng.standard_normal((1, DIM)).astype(np.float32))
    idx = np.zeros((layers, TOPK), np.int32)
    wgt = np.zeros((layers, TOPK), np.float32)
    for l in range(layers):
        i, w = topk_routing(rng, 1, E, TOPK)
        idx[l], wgt[l] = i[0], w[0]
    dx, di, dw = (hip.DevBuf.from_array(a) for a in (x, idx, wgt))
    dy = hip.DevBuf(layers * DIM * 4)
    wsp = hip.DevBuf(L.apus_hip_moe_workspace(st8, 1, TOPK))

    def run():
        for l in range(layers):
            hip._check(L.apus_hip_moe_routed_dev(st8, l, dx.ptr, di.ptr + l * TOPK * 4,
                                                 dw.ptr + l * TOPK * 4, 1, TOPK, LIMIT,
                                                 dy.ptr + l * DIM * 4, wsp.ptr), "routed_dev")

    run()
    eager = dy.to_array(np.float32, (layers, DIM)).copy()
    hip._check(L.apus_hip_graph_begin(), "graph_begin")
    run()
    hip._check(L.apus_hip_graph_end(), "graph_end")
    for rep in range(3):
        hip._check(L.apus_hip_memset(dy.ptr, 0, layers * DIM * 4), "memset")
        hip._check(L.apus_hip_graph_replay(1), "replay")
        hip._check(L.apus_hip_synchronize(), "sync")
        got = dy.to_array(np.float32, (layers, DIM))
        assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), rep
        run()                                        # eager launches between replays
        hip._check(L.apus_hip_synchronize(), "sync")
    assert _faults(hip) == 0


def test_layer1_barrier_timeout_poisons_output(hip, st8):
    """A barrier wait that gives up never hands back a finite wrong result.

    The host sets the wait's bound to zero polls, so every workgroup that
    reaches its wait before the release gives up at once (the 64 workgroups
    without phase-1 units arrive at the start and always do); every kernel
    still exits normally. Each workgroup that gave up writes NaN into its 16
    columns of y, the others (which saw the release, so every h code was
    written) equal the two-launch result bit for bit; apus_hip_synchronize
    returns nonzero naming the fault, the count reads back as the number of
    NaN column blocks, and with the default bound the next launch is clean.
    """
    _layer1_available(hip)
    L = hip.lib()
    rng = np.random.default_rng(6)
    x = bf16(rng.standard_normal((1, DIM)).astype(np.float32))
    idx, wgt = topk_routing(rng, 1, E, TOPK)
    assert L.apus_hip_layer1(0, None) == 0
    ref = _routed(hip, st8, 2, x, idx, wgt)[0]
    assert L.apus_hip_layer1(1, None) == 1
    assert _faults(hip) == 0
    dx, di, dw = (hip.DevBuf.from_array(np.ascontiguousarray(a)) for a in (x, idx, wgt))
    dy = hip.DevBuf(DIM * 4)
    wsp = hip.DevBuf(L.apus_hip_moe_workspace(st8, 1, TOPK))
    hip._check(L.apus_hip_layer1_spin_limit(0), "spin_limit")
    try:
        hip._check(L.apus_hip_moe_routed_dev(st8, 2, dx.ptr, di.ptr, dw.ptr, 1, TOPK, LIMIT,
                                             dy.ptr, wsp.ptr), "routed_dev")
        rc = L.apus_hip_synchronize()
        msg = L.apus_hip_last_error().decode()
    finally:
        hip._check(L.apus_hip_layer1_spin_limit(1 << 23), "spin_limit")
    assert rc != 0 and "gave up waiting" in msg, (rc, msg)
    y = dy.to_array(np.float32, (1, DIM))
    nanblk = np.isnan(y.reshape(DIM // 16, 16))
    assert (nanblk.all(1) | ~nanblk.any(1)).all()     # whole 16-column blocks
    nb = int(nanblk.all(1).sum())
    assert nb >= 64, nb                               # at least the workgroups without units
    ok = ~np.isnan(y)
    assert np.array_equal(y[ok].view(np.uint32), ref[ok].view(np.uint32))
    f = _faults(hip)
    print(f"timed-out workgroups: {f}, NaN column blocks: {nb}")
    assert f == nb
    # the default bound again: clean, bit-identical to the two launches
    hip._check(L.apus_hip_moe_routed_dev(st8, 2, dx.ptr, di.ptr, dw.ptr, 1, TOPK, LIMIT,
                                         dy.ptr, wsp.ptr), "routed_dev")
    hip._check(L.apus_hip_synchronize(), "sync")
    y = dy.to_array(np.float32, (1, DIM))
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))
    assert _faults(hip) == 0
