"""Decoded weight values are bit-exact on the GPU.

The matrix cores consume the stored E2M1 / E4M3 codes and E8M0 scales
directly. With a one-hot activation (code 1.0 at position k, scale 1), output
o of the GEMM is exactly weight[o, k] dequantised, so every code and scale
byte can be compared bit for bit with the oracle's decode
(orc_fp4_dequant_row / orc_e4m3_dequant, themselves pinned exhaustively
against the reference's apus_fp4_dequant_row_scalar / apus_e4m3_dequant_f32).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ONE = 0x38      # E4M3 code of 1.0


def onehot_acts(K, ks):
    codes = np.zeros((len(ks), K), np.uint8)
    for i, k in enumerate(ks):
        codes[i, k] = ONE
    return codes, np.ones((len(ks), K // 128), np.float32)


def test_fp4_decode_every_code_and_scale(hip, oracle):
    K, O = 128, 256
    # row o: byte pattern covering all 256 byte values (both nibbles) in
    # positions 0..31, scale byte = o (0..250: 6 * 2^(b-127) stays finite)
    w = np.zeros((O, K // 2), np.uint8)
    w[:, :16] = (np.arange(16)[None, :] * 16 + np.arange(16)[None, :]) % 256
    w[:, 16:32] = np.arange(256, dtype=np.uint8).reshape(16, 16)[np.arange(O) % 16]
    ws = np.zeros((O, K // 32), np.uint8)
    ws[:, 0] = np.minimum(np.arange(O), 250)
    ws[:, 1] = np.minimum(np.arange(O), 250)
    ks = list(range(64))
    codes, scales = onehot_acts(K, ks)
    got = hip.fp4_gemm(w, ws, codes, scales)           # [len(ks), O]
    for o in range(O):
        want = oracle.fp4_dequant_row(w[o].copy(), ws[o].copy())[:64]
        assert np.array_equal(got[:, o].view(np.uint32) & 0x7FFFFFFF,
                              want.view(np.uint32) & 0x7FFFFFFF), o
        # signs agree except for the zero codes (+0 vs -0 are the same value)
        nz = want != 0
        assert np.array_equal(np.signbit(got[nz, o]), np.signbit(want[nz]))


def test_fp8_decode_every_code(hip, oracle):
    K, O = 128, 256
    codes_w = np.arange(256, dtype=np.uint8)
    codes_w[0x7F] = 0x7E                 # the NaN codes are outside the contract
    codes_w[0xFF] = 0xFE
    w = np.zeros((O, K), np.uint8)
    w[:, 0] = codes_w                    # row o holds code o at k = 0
    w[:, 1] = codes_w[::-1]
    ws = np.full((O // 128, 1), 127, np.uint8)
    ws[1, 0] = 120                       # second row tile scaled by 2^-7
    codes, scales = onehot_acts(K, [0, 1])
    got = hip.fp8_gemm(w, ws, codes, scales)
    for o in range(O):
        for i, k in enumerate((0, 1)):
            want = np.float32(oracle.e4m3_dequant(int(w[o, k])) * oracle.ue8m0(int(ws[o // 128, 0])))
            assert abs(got[i, o]) == abs(want) and (want == 0 or np.sign(got[i, o]) == np.sign(want)), (o, k)


def test_hw_e4m3_conversion_exhaustive(hip):
    """The hardware E4M3 conversion that quantises activations inside the
    one-token MoE kernels equals the integer round-to-nearest-even encoder
    (itself equal to the reference's apus_e4m3_quant_f32 for all 2^32
    inputs, on the host) for every fp32 input with |x| <= 448."""
    import ctypes as C
    bad, last = C.c_uint(), C.c_uint()
    hip._check(hip.lib().apus_hip_check_e4m3_hw(C.byref(bad), C.byref(last)), "check")
    assert bad.value == 0, f"{bad.value} mismatches, e.g. bits {last.value:#010x}"
