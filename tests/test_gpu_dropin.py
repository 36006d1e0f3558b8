"""Drop-in through the reference's own call sites.

apus's hook table `apus_backend_hooks` (c/attn.h:203) lives in the
reference build (oracle/_ref/libapus_ref.so, compiled from the apus sources
in place). The test copies the backend's table (apus_hip_hooks(): its first
three members are ApusBackendHooks, c/backend_metal.h:73-80) into it as an
engine's enable path would (c/apus.c:155-166 does the same for Metal), then
calls the reference's own
functions:
  apus_fp8_linear  (hook tried first, c/attn.h:408-414)
  apus_bf16_linear (f32_linear hook with R_IN | R_OUT, c/attn.h:621-626)
  apus_head_gemv   (head_gemv hook, c/model.h:638-644)
and checks that the backend ran (apus_hip_dispatches grows) and that each
output is within the bar of the corresponding direct test. With the table
cleared again the same calls run the CPU kernels (dispatch count
unchanged). The table is always restored, since other tests use the
reference build as their checker.
"""
import ctypes as C

import numpy as np
import pytest

from helpers import acts, bf16, bf16_linear_ok, fp8_weights

pytestmark = pytest.mark.gpu


class BackendHooks(C.Structure):
    """c/backend_metal.h:73-80"""
    _fields_ = [("fp8_linear", C.c_void_p), ("f32_linear", C.c_void_p), ("head_gemv", C.c_void_p)]


@pytest.fixture
def hooked(hip, ref):
    table = BackendHooks.in_dll(ref.L, "apus_backend_hooks")
    saved = (table.fp8_linear, table.f32_linear, table.head_gemv)
    mine = hip.lib().apus_hip_hooks().contents
    table.fp8_linear, table.f32_linear, table.head_gemv = (mine.fp8_linear, mine.f32_linear,
                                                           mine.head_gemv)
    assert table.fp8_linear and table.f32_linear and table.head_gemv
    try:
        yield table
    finally:
        table.fp8_linear, table.f32_linear, table.head_gemv = saved


def _fp8_linear_via_reference(hip, ref, w, ws, x):
    M, K = x.shape
    O = w.shape[0]
    W = hip.fp8_weight(w, ws)
    out = np.empty((M, O), np.float32)
    f = ref.L.apus_fp8_linear
    f.restype = None
    f.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int]
    f(C.addressof(W), x.ctypes.data, out.ctypes.data, M, K, O)
    return out


def test_fp8_linear_through_reference_call_site(hip, ref, oracle, hooked):
    rng = np.random.default_rng(11)
    O, K, M = 1024, 4096, 3
    w, ws = fp8_weights(rng, O, K)
    x = acts(rng, M, K)
    d0 = hip.lib().apus_hip_dispatches()
    got = _fp8_linear_via_reference(hip, ref, w, ws, x)
    assert hip.lib().apus_hip_dispatches() > d0, "the hook did not run"
    c, s = oracle.act_quant(bf16(x))
    truth, esc = oracle.fp8_truth(w, ws, c, s)
    assert bf16_linear_ok(got, truth, 1e-4 * esc).all()
    # cleared table: the reference's CPU kernel, bit-identical to the oracle
    hooked.fp8_linear = None
    d1 = hip.lib().apus_hip_dispatches()
    cpu = _fp8_linear_via_reference(hip, ref, w, ws, x)
    assert hip.lib().apus_hip_dispatches() == d1
    assert np.array_equal(cpu.view(np.uint32), oracle.fp8_linear(w, ws, x).view(np.uint32))


def test_bf16_linear_and_head_through_reference_call_sites(hip, ref, oracle, hooked):
    rng = np.random.default_rng(12)
    O, K, M = 384, 1024, 2
    w = bf16(rng.standard_normal((O, K)).astype(np.float32) * 0.05)
    x = acts(rng, M, K)
    out = np.empty((M, O), np.float32)
    f = ref.L.apus_bf16_linear
    f.restype = None
    f.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int]
    d0 = hip.lib().apus_hip_dispatches()
    f(w.ctypes.data, x.ctypes.data, out.ctypes.data, M, K, O)
    assert hip.lib().apus_hip_dispatches() > d0
    truth, esc = oracle.wlinear_truth(w, x, 3)
    assert bf16_linear_ok(out, truth, 1e-5 * esc).all()
    # head GEMV over a BF16 view (c/model.h:638)
    Oh = 1000
    wh = (bf16(rng.standard_normal((Oh, K)).astype(np.float32)).view(np.uint32) >> 16).astype(np.uint16)
    t = hip.StTensor()
    t.name = b"head"
    t.dtype = 4                               # APUS_ST_BF16
    t.ndim = 2
    t.shape[0], t.shape[1] = Oh, K
    t.data = wh.ctypes.data
    t.nbytes = wh.nbytes
    yh = np.empty(Oh, np.float32)
    g = ref.L.apus_head_gemv
    g.restype = None
    g.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64]
    d1 = hip.lib().apus_hip_dispatches()
    g(C.addressof(t), x[0].ctypes.data, yh.ctypes.data, Oh, K)
    assert hip.lib().apus_hip_dispatches() > d1
    ht, he = oracle.wlinear_truth(wh, x[:1], 4)
    assert np.all(np.abs(yh.astype(np.float64) - ht[0]) <= 1e-5 * he[0] + 1e-30)
