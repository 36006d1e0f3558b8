"""Plain-weight linears on the GPU (f32_linear and head_gemv hooks,
apus_hip_wlinear_dev) against the oracle's restatement of apus_f32_linear /
apus_bf16_linear / apus_head_gemv (pinned bitwise against the reference).

The device sums each row in a strided order plus a shuffle tree where the
CPU sums sequentially, so unrounded outputs are checked with the err/esc
metric (|got - truth| <= 1e-5 * sum |w x|, truth in float64) and against the
oracle within 1e-4 max-rel; BF16-rounded outputs within one BF16 ulp of the
oracle's unrounded value plus 1e-5 * esc (a sum near a rounding boundary may
round the other way).
"""
import ctypes as C

import numpy as np
import pytest

from helpers import err_esc, max_rel

pytestmark = pytest.mark.gpu


def _data(rng, M, K, O, bf16w):
    w = (rng.standard_normal((O, K)) / np.sqrt(K)).astype(np.float32)
    if bf16w:
        w = (w.view(np.uint32) >> 16).astype(np.uint16)
    x = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    return w, x


def _check(got, oracle, w, x, flags):
    truth, esc = oracle.wlinear_truth(w, x, flags & ~2)
    if flags & 2:
        unr = oracle.wlinear(w, x, flags & ~2).astype(np.float64)
        ulp = np.abs(unr) * 2.0 ** -7
        assert np.all(np.abs(got - unr) <= ulp + 1e-5 * esc)
        assert np.array_equal(got, (got.view(np.uint32) & 0xFFFF0000).view(np.float32))
    else:
        assert err_esc(got, truth, esc) <= 1e-5
        assert max_rel(got, oracle.wlinear(w, x, flags)) <= 1e-4


@pytest.mark.parametrize("M,K,O,flags", [(1, 4096, 256, 0), (3, 4096, 1000, 3), (1, 4096, 1024, 6),
                                         (8, 1000, 77, 0), (20, 512, 64, 3), (2, 8, 5, 4),
                                         (1, 4096, 333, 7), (1, 2048, 70, 5), (1, 8192, 129, 6),
                                         (1, 1024, 40, 4)])
def test_f32_linear_hook(hip, oracle, rng, M, K, O, flags):
    w, x = _data(rng, M, K, O, flags & 4)
    got = hip.f32_linear(w, x, flags)
    _check(got, oracle, w, x, flags)


@pytest.mark.parametrize("bf16w,O,K", [(True, 4999, 4096), (False, 300, 2048), (True, 1027, 2048),
                                       (True, 515, 8192)])
def test_head_gemv_hook(hip, oracle, rng, bf16w, O, K):
    w, x = _data(rng, 1, K, O, bf16w)
    got = hip.head_gemv(w, x[0])
    _check(got[None, :], oracle, w, x, 4 if bf16w else 0)


def test_wlinear_dev_matches_hook(hip, rng):
    """The device-pointer entry runs the same kernel: bitwise equal to the
    host hook on the same data."""
    M, K, O, flags = 4, 2048, 300, 6
    w, x = _data(rng, M, K, O, True)
    L = hip.lib()
    dw, dx = hip.DevBuf.from_array(w), hip.DevBuf.from_array(x)
    do = hip.DevBuf(M * O * 4)
    hip._check(L.apus_hip_wlinear_dev(dw.ptr, dx.ptr, do.ptr, M, K, O, flags), "wlinear_dev")
    hip._check(L.apus_hip_synchronize(), "sync")
    got = do.to_array(np.float32, (M, O))
    assert np.array_equal(got.view(np.uint32), hip.f32_linear(w, x, flags).view(np.uint32))


def test_f32_linear_rejects_ragged_k(hip, rng):
    """K not a multiple of 8 is unsupported: the hook returns nonzero (the
    engine then runs its CPU kernel) and nothing is launched."""
    w, x = _data(rng, 1, 12, 4, False)
    L = hip.lib()
    out = np.empty((1, 4), np.float32)
    rc = L.apus_hip_f32_linear(w.ctypes.data, x.ctypes.data_as(hip.f32p),
                               out.ctypes.data_as(hip.f32p), 1, 12, 4, 0)
    assert rc != 0


def test_head_gemv_full_size(hip, oracle):
    """The LM head at the model's shape, BF16 [129280, 4096] (1.06 GB):
    every output row against the oracle would take the CPU minutes, so the
    first and last 256 rows (the last workgroup covers a partial 16-row
    block: 129280 = 16 * 8080) and 1024 seeded rows in between are checked,
    each output row depending on its own weight row only."""
    O, K = 129280, 4096
    rng = np.random.default_rng(17)
    # BF16 bits of N(0, 1/K) weights, generated in blocks to bound host memory
    w = np.empty((O, K), np.uint16)
    for r0 in range(0, O, 16384):
        r1 = min(O, r0 + 16384)
        blk = (rng.standard_normal((r1 - r0, K), dtype=np.float32) / np.float32(64.0))
        w[r0:r1] = (blk.view(np.uint32) >> 16).astype(np.uint16)
    x = (rng.standard_normal(K) * 2).astype(np.float32)
    got = hip.head_gemv(w, x)
    rows = np.unique(np.concatenate([np.arange(256), np.arange(O - 256, O),
                                     rng.choice(O, 1024, replace=False)]))
    _check(got[None, rows], oracle, w[rows], x[None, :], 4)
