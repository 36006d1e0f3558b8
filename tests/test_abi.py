"""C-ABI checks that need no GPU.

* libapus_hip.so loads and exports every entry point include/apus_hip.h
  declares, and the Python binding declares exactly that set;
* the host twins of the device numerics (compiled from the same inline
  source the kernels use) agree with the oracle on all 2^32 inputs;
* without a GPU, enable fails soft with a message and leaves the hooks NULL.
"""
import concurrent.futures as cf
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "apus_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(apus_hip_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    for must in ("apus_hip_enable", "apus_hip_disable", "apus_hip_is_enabled",
                 "apus_hip_fp4_linear", "apus_hip_fp8_linear", "apus_hip_moe_routed",
                 "apus_hip_fp4_gemm_grouped", "apus_hip_act_quant", "apus_hip_fp4_gemm",
                 "apus_hip_fp8_gemm"):
        assert must in syms


def test_library_exports_every_declared_symbol():
    import apus_hip
    lib = apus_hip.lib()
    for s in declared_symbols():
        assert hasattr(lib, s), s
    out = subprocess.run(["nm", "-D", "--defined-only", apus_hip.LIB_PATH],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (apus_hip_\w+)", out))
    assert set(declared_symbols()) <= exported
    assert set(apus_hip.SIGNATURES) == set(declared_symbols())


def _pin(oracle, which, fn):
    step = (1 << 32) // 8
    ptr = C.cast(fn, C.c_void_p)
    with cf.ThreadPoolExecutor(8) as ex:
        res = list(ex.map(lambda i: oracle.pin_unary(which, ptr, i * step, (i + 1) * step),
                          range(8)))
    return sum(r[0] for r in res)


def test_device_numerics_host_twins_exhaustive(oracle):
    import apus_hip
    lib = apus_hip.lib()
    assert _pin(oracle, 0, lib.apus_hip_host_bf16_round) == 0
    assert _pin(oracle, 1, lib.apus_hip_host_e4m3_quant) == 0


def test_device_act_scale_twin(oracle, rng):
    import apus_hip
    lib = apus_hip.lib()
    amaxes = np.concatenate([np.abs(rng.standard_normal(3000)) * 10.0 ** rng.integers(-6, 6, 3000),
                             [0.0, 1e-4, 1e-5, 448.0, 448.0 * 2 ** 3, 448.0 * 2 ** 3 * (1 + 2 ** -23)]])
    for a in amaxes.astype(np.float32):
        row = np.zeros(128, np.float32)
        row[17] = a
        _, sc = oracle.act_quant_row(row)
        assert lib.apus_hip_host_act_scale(float(a)) == sc[0], a


def test_enable_fails_soft_without_gpu():
    import apus_hip
    lib = apus_hip.lib()
    if os.path.exists("/dev/kfd") and os.access("/dev/kfd", os.R_OK | os.W_OK):
        pytest.skip("a GPU device node is present")
    err = C.create_string_buffer(256)
    assert lib.apus_hip_enable(err, 256) != 0
    assert err.value
    assert lib.apus_hip_is_enabled() == 0
    hooks = lib.apus_hip_hooks().contents
    assert all(getattr(hooks, f) is None for f in apus_hip.HOOK_FIELDS)
    # every host entry point reports "unsupported" instead of crashing
    x = np.zeros((1, 128), np.float32)
    codes = np.zeros((1, 128), np.uint8)
    sc = np.zeros((1, 1), np.float32)
    assert lib.apus_hip_act_quant(x.ctypes.data_as(apus_hip.f32p), 1, 128,
                                  codes.ctypes.data_as(apus_hip.u8p),
                                  sc.ctypes.data_as(apus_hip.f32p)) != 0
