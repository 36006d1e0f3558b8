/*
 * apus_numerics.h — bit-level numerics shared by the host and gfx950 device
 * code of the HIP backend: BF16 rounding, E4M3 encode, the per-128
 * power-of-two activation scale and E8M0 scale bytes.
 *
 * These are the rules of apus's activation quantisation
 * (c/fp4.h:219-321, c/attn.h:393-403), implemented in integer arithmetic so
 * that the device results are bit-identical to the CPU rules for every
 * input. The same inline functions are compiled for the host and exported
 * from libapus_hip.so (apus_hip_host_*), so they can be checked exhaustively
 * without a GPU.
 */
#ifndef APUS_NUMERICS_H
#define APUS_NUMERICS_H

#include <stdint.h>

#define APUS_HD __host__ __device__ __forceinline__

APUS_HD uint32_t apus_f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
APUS_HD float apus_u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

/* fp32 -> bf16 (round to nearest, ties to even), returned as fp32.
 * NaN is returned unchanged (c/fp4.h:262-270). */
APUS_HD float apus_bf16_rne(float x) {
    uint32_t u = apus_f2u(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return x;
    u += 0x7fffu + ((u >> 16) & 1u);
    return apus_u2f(u & 0xffff0000u);
}

/* fp32 -> E4M3 code (c/fp4.h:219-253): saturating clamp to +-448, then
 * round to nearest even on the E4M3 grid. For |x| >= 2^-6 the rounding is
 * done on the fp32 bits, keeping three mantissa bits (a carry walks into the
 * exponent on its own); the code is the kept bits re-biased from 127 to 7.
 * Below 2^-6 the grid is uniform with quantum 2^-9, so the code is
 * |x| * 512 (exact) rounded to the nearest even integer, 0..8.
 * Input must not be NaN. */
APUS_HD uint32_t apus_e4m3_code(float x) {
    x = x > 448.0f ? 448.0f : x;
    x = x < -448.0f ? -448.0f : x;
    uint32_t u = apus_f2u(x);
    uint32_t sign = (u >> 24) & 0x80u;
    uint32_t a = u & 0x7fffffffu;
    uint32_t code;
    if (a >= 0x3c800000u) {
        code = ((a + 0x7ffffu + ((a >> 20) & 1u)) >> 20) - (120u << 3);
    } else {
        code = (uint32_t)__builtin_rintf(apus_u2f(a) * 512.0f);
    }
    return sign | code;
}

/* Per-128 activation scale from the group's |max| (c/fp4.h:300-317):
 * amax floored at 1e-4, p = amax * fl(1/448), s = 2^ceil(log2 p) taken from
 * p's bits (biased exponent, plus one when any mantissa bit is set).
 * Returns the biased exponent of s, which is also s's E8M0 byte. */
APUS_HD uint32_t apus_act_scale_exp(float amax) {
    amax = amax < 1e-4f ? 1e-4f : amax;
    uint32_t pb = apus_f2u(amax * (1.0f / 448.0f));
    return ((pb >> 23) & 0xffu) + ((pb & 0x7fffffu) ? 1u : 0u);
}

/* Power of two with biased exponent e (1..254) as fp32. */
APUS_HD float apus_pow2_from_exp(uint32_t e) { return apus_u2f(e << 23); }

/* Reciprocal of that power of two, 2^(127-e); exact while 1 <= e <= 253.
 * An activation scale exponent is at most 247 for finite input (amax <=
 * FLT_MAX) and 255 when the group holds an infinity (the reference's scale
 * is then +inf, c/fp4.h:300-317): 0 is returned for e >= 254, so every
 * finite element quantises to a signed zero as x / inf does, and the E8M0
 * byte 255 makes the matrix cores return NaN for the row. */
APUS_HD float apus_inv_pow2_from_exp(uint32_t e) { return e >= 254u ? 0.0f : apus_u2f((254u - e) << 23); }

/* E8M0 byte of a power-of-two fp32 scale (its biased exponent). */
APUS_HD uint32_t apus_e8m0_of(float s) { return (apus_f2u(s) >> 23) & 0xffu; }

#endif /* APUS_NUMERICS_H */
