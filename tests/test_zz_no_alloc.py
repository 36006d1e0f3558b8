"""The allocation-free routed dispatch (apus_hip_moe_routed_dev_noalloc),
through the C ABI: two calls in a row, the second with fewer tokens, each
bit-identical to apus_hip_moe_routed_dev with a caller workspace (the same
kernels over the same workspace layout); a call whose workspace would not
fit the static scratch is refused without running, and so is a call with a
concurrency lane other than lane 0 selected (two lanes' calls would share
the one static workspace)."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

DIM, INTER, E, TOPK = 4096, 2048, 64, 6


def _routing(rng, s):
    idx = np.stack([rng.choice(E, TOPK, replace=False) for _ in range(s)]).astype(np.int32)
    w = rng.random((s, TOPK)).astype(np.float32)
    return idx, (w / w.sum(1, keepdims=True)).astype(np.float32)


def test_noalloc_matches_workspace_entry(hip):
    L = hip.lib()
    err = C.create_string_buffer(256)
    st = L.apus_hip_store_create(1, E, DIM, INTER, err, 256)
    assert st, err.value
    try:
        hip._check(L.apus_hip_store_fill_random(st, 8), "fill")
        rng = np.random.default_rng(9)
        # sorted pipeline (40 x 6 = 240 pairs), then the one-token kernels (3 x 6 = 18 pairs)
        for s in (40, 3):
            x = (rng.standard_normal((s, DIM)).astype(np.float32).view(np.uint32)
                 & 0xFFFF0000).view(np.float32)
            idx, wgt = _routing(rng, s)
            dx, di, dw = (hip.DevBuf.from_array(a) for a in (x, idx, wgt))
            y0, y1 = hip.DevBuf(s * DIM * 4), hip.DevBuf(s * DIM * 4)
            wsp = hip.DevBuf(L.apus_hip_moe_workspace(st, s, TOPK))
            assert L.apus_hip_moe_workspace(st, s, TOPK) <= L.apus_hip_moe_noalloc_max()
            hip._check(L.apus_hip_moe_routed_dev(st, 0, dx.ptr, di.ptr, dw.ptr, s, TOPK, 10.0,
                                                 y0.ptr, wsp.ptr), "routed_dev")
            hip._check(L.apus_hip_moe_routed_dev_noalloc(st, 0, dx.ptr, di.ptr, dw.ptr, s, TOPK,
                                                         10.0, y1.ptr), "routed_dev_noalloc")
            a = y0.to_array(np.float32, (s, DIM))
            b = y1.to_array(np.float32, (s, DIM))
            assert np.isfinite(a).all()
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), s
        # too large for the static scratch: refused, nothing launched
        s = 2048
        assert L.apus_hip_moe_workspace(st, s, TOPK) > L.apus_hip_moe_noalloc_max()
        d0 = L.apus_hip_dispatches()
        rc = L.apus_hip_moe_routed_dev_noalloc(st, 0, dx.ptr, di.ptr, dw.ptr, s, TOPK, 10.0, y1.ptr)
        assert rc != 0 and b"static scratch" in L.apus_hip_last_error()
        assert L.apus_hip_dispatches() == d0
        # a lane other than lane 0: refused, nothing launched
        hip._check(L.apus_hip_lanes(2), "lanes")
        hip._check(L.apus_hip_lane(1), "lane 1")
        try:
            s = 3
            rc = L.apus_hip_moe_routed_dev_noalloc(st, 0, dx.ptr, di.ptr, dw.ptr, s, TOPK, 10.0, y1.ptr)
            assert rc != 0 and b"lane 0 only" in L.apus_hip_last_error()
            assert L.apus_hip_dispatches() == d0
        finally:
            hip._check(L.apus_hip_lane(0), "lane 0")
    finally:
        L.apus_hip_store_free(st)
