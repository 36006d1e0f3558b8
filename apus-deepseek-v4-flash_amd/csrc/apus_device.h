/*
 * apus_device.h — gfx950 building blocks for the HIP backend: the
 * block-scaled F8F6F4 MFMA wrapper, 128-bit loads, wave reductions.
 *
 * MFMA operand layout (v_mfma_scale_f32_16x16x128_f8f6f4, CDNA4): lane l
 * holds row (l % 16) of A and column (l % 16) of B, and within that row /
 * column the 32 consecutive K elements of sub-block (l / 16); each lane also
 * supplies the E8M0 scale of its own 32-element sub-block (one byte of a
 * 32-bit register, picked by op_sel). FP8 operands take 32 bytes per lane,
 * FP4 operands 16 bytes (two E2M1 per byte, low nibble first). The result
 * D[i][j] = sum_k A[i][k] B[k][j] lands in lane l as D[4*(l/16) + q][l % 16],
 * q = 0..3. The K order inside one instruction is irrelevant to the result
 * set, so the kernels are free to choose which 32-element groups of the
 * reduction dimension feed which lane group.
 */
#ifndef APUS_DEVICE_H
#define APUS_DEVICE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "apus_numerics.h"

typedef int   apus_v8i __attribute__((ext_vector_type(8)));
typedef float apus_v4f __attribute__((ext_vector_type(4)));

/* operand format codes of the F8F6F4 MFMA (cbsz for A, blgp for B) */
#define APUS_FMT_E4M3 0
#define APUS_FMT_E2M1 4

/* One 16x16x128 block-scaled MFMA. AF/BF: operand formats; SA/SB: which byte
 * of the scale registers holds this lane's E8M0 scale. */
template <int AF, int BF, int SA, int SB>
__device__ __forceinline__ apus_v4f apus_mfma_scaled(apus_v8i a, apus_v8i b,
                                                     apus_v4f c, int sa, int sb) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, AF, BF, SA, sa, SB, sb);
}

/* Loads through global-address-space pointers. Pointers read from memory
 * (entry tables) are generic, and a generic load is a flat load, which the
 * hardware counts against both the vector-memory and the LDS counters: every
 * LDS wait would then also wait for the weight prefetch ring. */
#define APUS_GLOBAL __attribute__((address_space(1)))

template <typename T>
__device__ __forceinline__ T apus_gld(const void *p) {
    /* raw chunks of the object's size, then a bit cast (class types cannot
     * be copy-constructed from an address-space-qualified reference) */
    if constexpr (sizeof(T) == 16) {
        typedef unsigned v4 __attribute__((ext_vector_type(4)));
        return __builtin_bit_cast(T, *(const APUS_GLOBAL v4 *)p);
    } else if constexpr (sizeof(T) == 8) {
        return __builtin_bit_cast(T, *(const APUS_GLOBAL unsigned long long *)p);
    } else if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, *(const APUS_GLOBAL unsigned *)p);
    } else if constexpr (sizeof(T) == 1) {
        return __builtin_bit_cast(T, *(const APUS_GLOBAL unsigned char *)p);
    } else {
        static_assert(sizeof(T) % 8 == 0, "apus_gld size");
        struct Raw { unsigned long long d[sizeof(T) / 8]; } r;
#pragma unroll
        for (unsigned i = 0; i < sizeof(T) / 8; ++i)
            r.d[i] = ((const APUS_GLOBAL unsigned long long *)p)[i];
        return __builtin_bit_cast(T, r);
    }
}

template <typename T>
__device__ __forceinline__ void apus_gst(void *p, T v) {
    *(APUS_GLOBAL T *)p = v;
}

__device__ __forceinline__ uint4 apus_ld16(const uint8_t *p) {
    return apus_gld<uint4>(p);
}

typedef unsigned apus_v4u __attribute__((ext_vector_type(4)));

/* streamed (read-once) 16-byte load: one global_load_dwordx4 with the
 * non-temporal hint, so weight slabs do not evict the activations that
 * every workgroup re-reads */
__device__ __forceinline__ apus_v4u apus_ld16_stream(const uint8_t *p) {
    return __builtin_nontemporal_load((const APUS_GLOBAL apus_v4u *)p);
}

__device__ __forceinline__ float apus_wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

/* The same maximum with DPP moves inside each 16-lane row (quad
 * permutations, half-row and row mirrors) and the four row results read
 * from lanes 0, 16, 32, 48; every lane must be active. fmaxf is
 * order-independent, so the result equals apus_wave_max's. */
template <int CTRL>
__device__ __forceinline__ float apus_dpp_max(float v) {
    const int o = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true);
    return fmaxf(v, __builtin_bit_cast(float, o));
}
__device__ __forceinline__ float apus_wave_max_dpp(float v) {
    v = apus_dpp_max<0xB1>(v);     /* quad_perm [1, 0, 3, 2] */
    v = apus_dpp_max<0x4E>(v);     /* quad_perm [2, 3, 0, 1] */
    v = apus_dpp_max<0x141>(v);    /* row_half_mirror */
    v = apus_dpp_max<0x140>(v);    /* row_mirror */
    const int b = __builtin_bit_cast(int, v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

/* h = bf16(silu(g') * u') with g' = min(g, limit), u' = clamp(u, +-limit)
 * when limit > 0 (c/moe.h:113-126); every step rounded as written. */
__device__ __forceinline__ float apus_swiglu_h(float g, float u, float limit) {
    if (limit > 0.0f) {
        u = u > limit ? limit : (u < -limit ? -limit : u);
        g = g > limit ? limit : g;
    }
    const float sig = 1.0f / (1.0f + expf(-g));
    return apus_bf16_rne((g * sig) * u);
}

/* Workgroup barrier for LDS hand-off only: waits for this wave's LDS
 * operations, not for its outstanding global loads. __syncthreads() also
 * fences global memory, i.e. waits for every load in flight (vmcnt 0), which
 * would drain a register prefetch ring at each barrier. */
__device__ __forceinline__ void apus_lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

/* 16-byte chunk slot of chunk c of a 128-byte activation row staged in LDS:
 * c ^ apus_row_swz(row). A fragment read (ds_read_b128, lane (r, g) reading
 * chunk g or 4 + g of row r, 16 rows) is then conflict-free on gfx950:
 * measured with the LDS counters, 4 cycles per read against 8 for the swizzle
 * (r ^ (r >> 3)) & 7 and 16 for none. */
__device__ __forceinline__ int apus_row_swz(int row) { return row & 7; }

/* Two or four E4M3 codes (bytes a, b[, c, d] in order) by the hardware conversion,
 * round-to-nearest-even. Equal to apus_e4m3_code for every fp32 input with
 * |x| <= 448 (checked exhaustively on the device by
 * apus_hip_check_e4m3_hw); callers pass values already scaled into that range
 * (activation groups: |v| / s <= 448 by the choice of s). */
__device__ __forceinline__ uint32_t apus_e4m3_pack2_hw(float a, float b) {
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xffffu;
}
__device__ __forceinline__ uint32_t apus_e4m3_pack4_hw(float a, float b, float c, float d) {
    const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
}

/* Expert choice of one token by a 256-thread workgroup (c/moe.h:384-410):
 * the stable descending top-k of the selection scores sel[0..E) (the
 * reference's repeated arg-max with strict greater-than: the lowest index
 * wins among equal scores, c/attn.h:668-686), or, with t2e, the hash table's
 * row t2e[0..topk). The arg-max scan picks experts in the order of the key
 * (score descending, index ascending), so expert e lands in slot rank(e) =
 * #{f : key(f) > key(e)} when that rank is below topk; key(e) = (order-
 * preserving bits of the score with -0 folded into +0, ~e) makes the
 * comparison one 64-bit compare. Leaves chosen[j] and its router score
 * chp[j] = sp[chosen[j]] in LDS for j < topk (visible after the final
 * barrier). Every thread of the workgroup must call it. E <= 1024. */
__device__ __forceinline__ void apus_route_token(const float *sel, const float *sp, int E, int topk,
                                                 const int64_t *t2e, uint64_t *lk, int32_t *chosen,
                                                 float *chp) {
    const int tid = threadIdx.x;
    if (t2e) {
        if (tid < topk) {
            const int e = (int)t2e[tid];
            chosen[tid] = e;
            chp[tid] = sp[e];
        }
    } else {
        const int E4 = (E + 3) >> 2;
        for (int e = tid; e < E4 * 4; e += 256) {
            uint64_t k = 0;
            if (e < E) {
                const uint32_t b = __float_as_uint(sel[e] + 0.0f);
                const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
                k = ((uint64_t)o << 32) | (uint32_t)~(uint32_t)e;
            }
            lk[e] = k;
        }
        __syncthreads();
        for (int e = tid; e < E; e += 256) {
            const uint64_t ke = lk[e];
            int rank = 0;
            for (int f2 = 0; f2 < E4 * 2; ++f2) {
                const ulonglong2 u = *reinterpret_cast<const ulonglong2 *>(lk + 2 * f2);
                rank += (int)(u.x > ke) + (int)(u.y > ke);
            }
            if (rank < topk) {
                chosen[rank] = e;
                chp[rank] = sp[e];
            }
        }
    }
    __syncthreads();
}

/* wgt[j] = chp[j] / sum_j' chp[j'] * route_scale, the sum in j order
 * (c/moe.h:400-410) */
__device__ __forceinline__ float apus_route_weight(const float *chp, int topk, int j,
                                                   float route_scale) {
    float sum = 0.0f;
    for (int i = 0; i < topk; ++i) sum += chp[i];
    return chp[j] / sum * route_scale;
}

#endif /* APUS_DEVICE_H */
