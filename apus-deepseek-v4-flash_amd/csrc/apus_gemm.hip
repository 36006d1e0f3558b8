/*
 * apus_gemm.hip — block-scaled GEMM kernels on the gfx950 F8F6F4 matrix cores:
 * E4M3 activations (quantised per 128 along K, E8M0 scales) against MXFP4
 * (E2M1 + E8M0 per 32) or FP8-E4M3 (E8M0 per 128x128 tile) weights.
 * Semantics: c/fp4.h:367-395 and c/fp8.h:191-218 (normative GEMMs),
 * c/fp4.h:936-986 (grouped entries over shared activation rows).
 *
 * Schedules, chosen by apus_launch_gemm:
 *  - split-K (apus_gemm_kernel): few row tiles, e.g. one dense GEMV; the
 *    waves of a workgroup split K and reduce through LDS.
 *  - decode (apus_gemm_decode_kernel): grouped launches of few-row entries
 *    (routed experts at decode); activations staged once in LDS, each wave
 *    streams a whole-K 16-row weight tile through a prefetch ring.
 *  - prefill (apus_gemm_prefill_kernel): grouped launches with many rows
 *    per entry; activation slices double-buffered in LDS, 4 token tiles per
 *    weight pass.
 *  - stream (apus_gemm_stream_kernel): other grouped shapes.
 * In all of them, every output is one accumulation chain over its 128-groups
 * in a fixed order, so results do not depend on M, on the position of a row
 * within its entry, or on timing.
 *
 * Build-time tuning constants (defaults are the measured best on gfx950;
 * -D overrides exist for measurements only): APUS_DEC_WAVES (decode
 * workgroup waves, 4), APUS_DEC_PD_FP4 (decode FP4 weight ring slices, 3),
 * APUS_PRE_WAVES (prefill workgroup waves, 8), APUS_PRE_PD4 (prefill FP4
 * ring slices, 2), APUS_PREFILL_ROWS (rows per many-row work item, 64),
 * APUS_TILE_TM (tile schedule token fragments per wave, 4), APUS_TILE_DA
 * (activation ring groups, 6), APUS_TILE_PDX (weight ring multiplier, 1).
 */
#include "apus_device.h"
#include "apus_internal.h"

/*
 * Tiling. A workgroup owns 16 consecutive weight rows (the 16 MFMA columns)
 * of one entry and all of that entry's rows (tokens) in tiles of 16. The
 * reduction dimension is cut into slices of 512; slice s belongs to wave
 * s % waves, so the waves of a workgroup split K and their partial 16x16
 * tiles are summed through LDS in a fixed wave order (the result does not
 * depend on timing, nor on M or on the position of a row in the entry).
 *
 * One MFMA covers exactly one 128-element K group (group q = 4s + step), so
 * the activation scale and, for FP8, the 128x128 weight tile scale are the
 * same for all 32-element blocks of the instruction. Operand placement
 * (measured on gfx950): an E4M3 operand lane of lane group g holds K
 * [16g, 16g+16) in bytes 0..15 and [64+16g, +16) in bytes 16..31; an E2M1
 * operand lane holds the contiguous K [32g, 32g+32); the E8M0 scale of
 * (row r, 32-block b) is taken from lane 16b + r. Hence per step:
 *   A (E4M3 codes) lane g: bytes [q*128 + 16g, +16) and [q*128 + 64 + 16g, +16)
 *   B E4M3 weights: the same two 16-byte pieces of weight row o
 *   B E2M1 weights: bytes [q*64 + 16g, +16) of row o, scale byte 4q + g
 * which makes each instruction read 64 contiguous bytes per weight row.
 */
template <int WF, bool GROUPED>
__global__ __launch_bounds__(512) void apus_gemm_kernel(ApusGemmArgs args) {
    __shared__ float red[8][16][17];
    const ApusGemmEnt ent = GROUPED ? apus_gld<ApusGemmEnt>(args.ents + blockIdx.y) : args.ent0;
    if (ent.M <= 0) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nw = blockDim.x >> 6;
    const int O = args.O, K = args.K;
    const int r = lane & 15, g = lane >> 4;
    const int o = blockIdx.x * 16 + r;
    const bool ovalid = o < O;
    const int nq = K >> 7;                 /* 128-groups */
    const int nslice = (nq + 3) >> 2;

    for (int t0 = 0; t0 < ent.M; t0 += 16) {
        apus_v4f acc = {0.f, 0.f, 0.f, 0.f};
        const int m = t0 + r;
        const bool mvalid = m < ent.M;
        const int arow = mvalid ? (ent.arows ? apus_gld<int>(ent.arows + (m)) : ent.a0 + m) : 0;
        for (int s = wave; s < nslice; s += nw) {
            apus_v8i bw[4], aw[4];
            int sbv[4], sav[4];
            /* FP4 weight scales of this slice: 16 bytes, byte 4*step + g */
            apus_v4u sw4 = {0x7f7f7f7fu, 0x7f7f7f7fu, 0x7f7f7f7fu, 0x7f7f7f7fu};
            if (WF == APUS_W_FP4 && ovalid) {
                if ((s + 1) * 4 <= nq) {
                    sw4 = apus_gld<apus_v4u>(ent.ws + (size_t)o * (K >> 5) + s * 16);
                } else {
                    for (int st = 0; st < 4; ++st)
                        if (s * 4 + st < nq)
                            sw4[st] = apus_gld<unsigned>(ent.ws + (size_t)o * (K >> 5) + (s * 4 + st) * 4);
                }
            }
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const int q = s * 4 + st;
                const bool qvalid = q < nq;
                /* B */
                if (WF == APUS_W_FP4) {
                    if (ovalid && qvalid) {
                        apus_v4u w = apus_ld16_stream(ent.w + (size_t)o * (K >> 1) + q * 64 + g * 16);
                        bw[st] = apus_v8i{(int)w.x, (int)w.y, (int)w.z, (int)w.w, 0, 0, 0, 0};
                    } else {
                        bw[st] = apus_v8i{0, 0, 0, 0, 0, 0, 0, 0};
                    }
                    sbv[st] = (int)((sw4[st] >> (8 * g)) & 0xffu);
                } else {
                    if (ovalid && qvalid) {
                        const uint8_t *p = ent.w + (size_t)o * K + q * 128 + g * 16;
                        apus_v4u w0 = apus_ld16_stream(p), w1 = apus_ld16_stream(p + 64);
                        bw[st] = apus_v8i{(int)w0.x, (int)w0.y, (int)w0.z, (int)w0.w,
                                          (int)w1.x, (int)w1.y, (int)w1.z, (int)w1.w};
                        sbv[st] = apus_gld<uint8_t>(ent.ws + ((size_t)(o >> 7) * nq + q));
                    } else {
                        bw[st] = apus_v8i{0, 0, 0, 0, 0, 0, 0, 0};
                        sbv[st] = 0x7f;
                    }
                }
                /* A */
                if (mvalid && qvalid) {
                    const uint8_t *p = args.acodes + (size_t)arow * K + q * 128 + g * 16;
                    uint4 a0 = apus_ld16(p), a1 = apus_ld16(p + 64);
                    aw[st] = apus_v8i{(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w,
                                      (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
                    sav[st] = (int)apus_e8m0_of(apus_gld<float>(args.ascale + ((size_t)arow * nq + q)));
                } else {
                    aw[st] = apus_v8i{0, 0, 0, 0, 0, 0, 0, 0};
                    sav[st] = 0x7f;
                }
            }
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                if (WF == APUS_W_FP4)
                    acc = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E2M1, 0, 0>(aw[st], bw[st], acc, sav[st], sbv[st]);
                else
                    acc = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E4M3, 0, 0>(aw[st], bw[st], acc, sav[st], sbv[st]);
            }
        }
        /* D[i][j]: i = token 4g+q of this tile, j = weight row r */
#pragma unroll
        for (int q = 0; q < 4; ++q) red[wave][4 * g + q][r] = acc[q];
        __syncthreads();
        for (int e = threadIdx.x; e < 256; e += blockDim.x) {
            const int i = e >> 4, j = e & 15;
            const int mm = t0 + i, oo = blockIdx.x * 16 + j;
            if (mm < ent.M && oo < O) {
                float v = red[0][i][j];
                for (int w = 1; w < nw; ++w) v += red[w][i][j];
                if (args.round_out) v = apus_bf16_rne(v);
                const int orow = ent.orows ? apus_gld<int>(ent.orows + (mm)) : ent.o0 + mm;
                apus_gst<float>(ent.out + ((size_t)orow * args.ldo + oo), v);
            }
        }
        __syncthreads();
    }
}

/*
 * Streaming variant for launches with many row tiles (grouped expert GEMMs):
 * every wave owns one 16-row tile over the whole K, so no cross-wave
 * reduction is needed; each output is a single accumulation chain over the
 * 128-groups in order q = 0, 1, ... (again independent of M and of the row's
 * position). The weight fragment of slice s+1 is loaded while slice s is
 * multiplied, and up to MT token tiles are accumulated per weight pass, so a
 * weight slab is streamed from HBM once per MT*16 tokens.
 * Operand placement as in apus_gemm_kernel.
 */
template <int WF>
struct ApusBFrag {
    apus_v4u w[4][WF == APUS_W_FP4 ? 1 : 2];
    apus_v4u s;       /* FP4: 16 group-scale bytes; FP8: byte st = tile scale */
};

template <int WF>
__device__ __forceinline__ void apus_load_b(ApusBFrag<WF> &f, const ApusGemmEnt &ent, int o,
                                            bool ovalid, int s, int nq, int K, int g) {
    const bool full = (s + 1) * 4 <= nq;
#pragma unroll
    for (int st = 0; st < 4; ++st) {
        const int q = s * 4 + st;
        const bool v = ovalid && q < nq;
        if (WF == APUS_W_FP4) {
            f.w[st][0] = v ? apus_ld16_stream(ent.w + (size_t)o * (K >> 1) + q * 64 + g * 16)
                           : apus_v4u{0u, 0u, 0u, 0u};
        } else {
            const uint8_t *p = ent.w + (size_t)o * K + q * 128 + g * 16;
            f.w[st][0] = v ? apus_ld16_stream(p) : apus_v4u{0u, 0u, 0u, 0u};
            f.w[st][1] = v ? apus_ld16_stream(p + 64) : apus_v4u{0u, 0u, 0u, 0u};
        }
    }
    if (WF == APUS_W_FP4) {
        if (ovalid && full) {
            f.s = apus_gld<apus_v4u>(ent.ws + (size_t)o * (K >> 5) + s * 16);
        } else {
#pragma unroll
            for (int st = 0; st < 4; ++st)
                f.s[st] = (ovalid && s * 4 + st < nq)
                    ? apus_gld<unsigned>(ent.ws + (size_t)o * (K >> 5) + (s * 4 + st) * 4)
                    : 0x7f7f7f7fu;
        }
    } else {
#pragma unroll
        for (int st = 0; st < 4; ++st)
            f.s[st] = (ovalid && s * 4 + st < nq) ? apus_gld<uint8_t>(ent.ws + ((size_t)(o >> 7) * nq + s * 4 + st)) : 0x7fu;
    }
}

template <int WF, int MT>
__global__ __launch_bounds__(256) void apus_gemm_stream_kernel(ApusGemmArgs args) {
    const ApusGemmEnt ent = apus_gld<ApusGemmEnt>(args.ents + blockIdx.y);
    if (ent.M <= 0) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int O = args.O, K = args.K;
    const int r = lane & 15, g = lane >> 4;
    const int tile = blockIdx.x * 4 + wave;
    if (tile * 16 >= O) return;
    const int o = tile * 16 + r;
    const bool ovalid = o < O;
    const int nq = K >> 7;
    const int nslice = (nq + 3) >> 2;

    for (int c0 = 0; c0 < ent.M; c0 += 16 * MT) {
        const int ntile = min(MT, (ent.M - c0 + 15) >> 4);
        apus_v4f acc[MT];
        int arow[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            acc[t] = apus_v4f{0.f, 0.f, 0.f, 0.f};
            const int m = c0 + t * 16 + r;
            arow[t] = m < ent.M ? (ent.arows ? apus_gld<int>(ent.arows + (m)) : ent.a0 + m) : -1;
        }
        ApusBFrag<WF> cur, nxt;
        apus_load_b<WF>(cur, ent, o, ovalid, 0, nq, K, g);
        for (int s = 0; s < nslice; ++s) {
            if (s + 1 < nslice) apus_load_b<WF>(nxt, ent, o, ovalid, s + 1, nq, K, g);
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                if (t >= ntile) break;
                const int ar = arow[t];
#pragma unroll
                for (int st = 0; st < 4; ++st) {
                    const int q = s * 4 + st;
                    apus_v8i a = apus_v8i{0, 0, 0, 0, 0, 0, 0, 0};
                    int sa = 0x7f;
                    if (ar >= 0 && q < nq) {
                        const uint8_t *p = args.acodes + (size_t)ar * K + q * 128 + g * 16;
                        const uint4 a0 = apus_ld16(p), a1 = apus_ld16(p + 64);
                        a = apus_v8i{(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w,
                                     (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
                        sa = (int)apus_e8m0_of(apus_gld<float>(args.ascale + ((size_t)ar * nq + q)));
                    }
                    if (WF == APUS_W_FP4) {
                        const apus_v4u w = cur.w[st][0];
                        const apus_v8i b = apus_v8i{(int)w.x, (int)w.y, (int)w.z, (int)w.w, 0, 0, 0, 0};
                        const int sb = (int)((cur.s[st] >> (8 * g)) & 0xffu);
                        acc[t] = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E2M1, 0, 0>(a, b, acc[t], sa, sb);
                    } else {
                        const apus_v4u w0 = cur.w[st][0], w1 = cur.w[st][1];
                        const apus_v8i b = apus_v8i{(int)w0.x, (int)w0.y, (int)w0.z, (int)w0.w,
                                                    (int)w1.x, (int)w1.y, (int)w1.z, (int)w1.w};
                        acc[t] = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E4M3, 0, 0>(a, b, acc[t], sa, (int)cur.s[st]);
                    }
                }
            }
            cur = nxt;
        }
        /* lane holds D[4g+q][r]: token c0 + 16t + 4g + q, weight row o */
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            if (t >= ntile) break;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int mm = c0 + t * 16 + 4 * g + q;
                if (mm < ent.M && ovalid) {
                    float v = acc[t][q];
                    if (args.round_out) v = apus_bf16_rne(v);
                    const int orow = ent.orows ? apus_gld<int>(ent.orows + (mm)) : ent.o0 + mm;
                    apus_gst<float>(ent.out + ((size_t)orow * args.ldo + o), v);
                }
            }
        }
    }
}

/*
 * Decode schedule. K = 512 * NS is a template constant and O % 16 == 0 (the
 * launcher checks), so the slice loop is straight-line code with no per-lane
 * bounds tests: a divergent branch or a loop back edge around the prefetch
 * ring makes the compiler drain every outstanding load (s_waitcnt vmcnt(0)),
 * which would empty the ring each step. The workgroup's four waves share one
 * entry; its activation rows (R at a time, whole K) are staged in LDS as
 * E4M3 codes and E8M0 bytes, rows beyond the entry are zeroed by a select.
 * The staged rows are either read as codes (ASRC CODES) or quantised while
 * staging from fp32 rows (F32: the act quant of c/attn.h:393-403; SWIGLU:
 * h = swiglu(g, u) then its act quant, c/moe.h:113-126 and :309-314), with
 * the same per-element steps as the standalone kernels, so the codes are
 * identical.
 */
#ifndef APUS_TILE_FP
#define APUS_TILE_FP 1
#endif
#ifndef APUS_DEC_WAVES
#define APUS_DEC_WAVES 4
#endif
#define APUS_DEC_NT (64 * APUS_DEC_WAVES)
#ifndef APUS_DEC_SC_UPFRONT
#define APUS_DEC_SC_UPFRONT 1
#endif

/* The weight stream of one lane of a 16-row tile: the address of its
 * 16 bytes of 128-group 0 and the distance between consecutive groups (qs)
 * and, for FP4, between the 16-byte scale runs of consecutive 512-slices
 * (ss). Row-major weights ([O, K/2] or [O, K]): 16 rows x 64 bytes per load.
 * MFMA-tiled weights (launch flag wtiled): for each 16-row tile and
 * 128-group the 64 lanes' pieces are stored back to back, so a load reads
 * 1 KB contiguously; FP4 scales are [O/16][K/512][16 rows][16 bytes]. FP8
 * takes its second 16-byte piece of a group at qs / 2 in both layouts. */
struct ApusWLane {
    const uint8_t *w, *s;
    uint32_t qs, ss;
};

template <int WF>
__device__ __forceinline__ ApusWLane apus_wlane(const ApusGemmEnt &ent, bool tiled, int o, int lane,
                                                int K) {
    const int NQ = K >> 7, NS = K >> 9;
    ApusWLane l;
    if constexpr (WF == APUS_W_FP4) {
        if (tiled) {
            l.w = ent.w + ((size_t)(o >> 4) * NQ * 64 + lane) * 16; l.qs = 1024;
            l.s = ent.ws + ((size_t)(o >> 4) * NS * 16 + (o & 15)) * 16; l.ss = 256;
        } else {
            l.w = ent.w + (size_t)o * (K >> 1) + (lane >> 4) * 16; l.qs = 64;
            l.s = ent.ws + (size_t)o * (K >> 5); l.ss = 16;
        }
    } else {
        if (tiled) { l.w = ent.w + ((size_t)(o >> 4) * NQ * 128 + lane) * 16; l.qs = 2048; }
        else       { l.w = ent.w + (size_t)o * K + (lane >> 4) * 16; l.qs = 128; }
        l.s = ent.ws + (size_t)(o >> 7) * NQ; l.ss = 4;
    }
    return l;
}

/* the four groups of 512-slice s of a lane's weight stream (and, unless
 * SC is false, the slice's scales) */
template <int WF, bool SC = true>
__device__ __forceinline__ void apus_load_b_full(ApusBFrag<WF> &f, const ApusWLane &l, int s) {
#pragma unroll
    for (int st = 0; st < 4; ++st) {
        const uint8_t *p = l.w + (size_t)(s * 4 + st) * l.qs;
        f.w[st][0] = apus_ld16_stream(p);
        if constexpr (WF == APUS_W_FP8) f.w[st][1] = apus_ld16_stream(p + (l.qs >> 1));
    }
    if constexpr (!SC) {
        return;
    } else if constexpr (WF == APUS_W_FP4) {
        f.s = apus_gld<apus_v4u>(l.s + (size_t)s * l.ss);
    } else {
        const unsigned b4 = apus_gld<unsigned>(l.s + s * 4);
        f.s = apus_v4u{b4 & 0xffu, (b4 >> 8) & 0xffu, (b4 >> 16) & 0xffu, b4 >> 24};
    }
}

/* weights of matrix slot `mat` of expert e: computed from a regular slab
 * layout, or read from the pointer tables */
__device__ __forceinline__ void apus_expert_ptrs(const ApusGemmArgs &a, int mat, int e,
                                                 const uint8_t *&w, const uint8_t *&ws) {
    if (a.pbase) {
        const uint8_t *b = a.pbase + (size_t)e * a.pstride;
        w = b + (mat ? a.pwoff[1] : a.pwoff[0]);
        ws = b + (mat ? a.psoff[1] : a.psoff[0]);
    } else {
        w = apus_gld<const uint8_t *>((mat ? a.pw[1] : a.pw[0]) + e);
        ws = apus_gld<const uint8_t *>((mat ? a.pws[1] : a.pws[0]) + e);
    }
}

/* the entry of launch row y: table, routed pair, or the single entry */
__device__ __forceinline__ ApusGemmEnt apus_entry_of(const ApusGemmArgs &a, int y) {
    if (a.ents) {
        /* y is uniform (the launch row): one batch of scalar loads for every
         * field (a vector load of the entry measured the same to 1 % slower
         * at configs 2 and 3) */
        const ApusGemmEnt e = a.ents[y];
        asm volatile("" ::"s"(e.w), "s"(e.ws), "s"(e.out), "s"(e.arows), "s"(e.orows), "s"(e.a0),
                     "s"(e.o0), "s"(e.M));
        return e;
    }
    if (!a.pidx) return y == 0 ? a.ent0 : a.ent1;
    ApusGemmEnt ent;
    const int p = y / a.nmat, mat = y - p * a.nmat;
    const int e = apus_gld<int>(a.pidx + p);
    const bool ok = (unsigned)e < (unsigned)a.pE;
    const int ee = ok ? e : 0;
    apus_expert_ptrs(a, mat, ee, ent.w, ent.ws);
    ent.out = mat ? a.pout[1] : a.pout[0];
    ent.arows = nullptr; ent.orows = nullptr;
    ent.a0 = p / a.adiv; ent.o0 = p; ent.M = ok ? 1 : 0; ent.pad = 0;
    return ent;
}

/* Quantising staging of activation rows into LDS (codes [R][K + 32], E8M0
 * bytes [R][K/128]). Eight lanes own one 128-group (16 elements each); a
 * wave covers 8 groups per pass, a pass 32 groups. The loads of a pass and
 * its quantisation are separate steps so that the first pass's loads can be
 * issued before the weight ring (and before the entry lookup when the row
 * is known without it). */
template <int ASRC>
struct ApusStageRaw {
    float4 g[4], u[4];
    int row, q;
    bool ok;
};

template <int K, int ASRC>
__device__ __forceinline__ void apus_stage_load(const ApusGemmArgs &a, const int *arows, int a0,
                                                int c0, int rows, int pass, ApusStageRaw<ASRC> &r) {
    constexpr int NQ = K / 128;
    const int sub = threadIdx.x & 7;
    /* rows * NQ is a multiple of 16, so this test is uniform over each wave */
    const int gi = pass * (APUS_DEC_NT / 8) + (threadIdx.x >> 3);
    r.ok = gi < rows * NQ;
    r.row = gi / NQ;
    r.q = gi - r.row * NQ;
    if (r.ok) {
        const int mm = c0 + r.row;
        const int ar = arows ? apus_gld<int>(arows + mm) : a0 + mm;
        const size_t off = (size_t)ar * K + r.q * 128 + sub * 16;
#pragma unroll
        for (int i = 0; i < 4; ++i) r.g[i] = apus_gld<float4>(a.ax + off + 4 * i);
        if constexpr (ASRC == APUS_A_SWIGLU) {
#pragma unroll
            for (int i = 0; i < 4; ++i) r.u[i] = apus_gld<float4>(a.au + off + 4 * i);
        }
    }
}

template <int K, int ASRC>
__device__ __forceinline__ void apus_stage_quant(const ApusGemmArgs &a, const ApusStageRaw<ASRC> &r,
                                                 uint8_t *lcodes, uint8_t *lsc) {
    constexpr int NQ = K / 128, LDK = K + 32;
    const int sub = threadIdx.x & 7;
    if (!r.ok) return;
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (ASRC == APUS_A_F32) {
            v[4 * i] = apus_bf16_rne(r.g[i].x); v[4 * i + 1] = apus_bf16_rne(r.g[i].y);
            v[4 * i + 2] = apus_bf16_rne(r.g[i].z); v[4 * i + 3] = apus_bf16_rne(r.g[i].w);
        } else {
            v[4 * i] = apus_swiglu_h(r.g[i].x, r.u[i].x, a.limit);
            v[4 * i + 1] = apus_swiglu_h(r.g[i].y, r.u[i].y, a.limit);
            v[4 * i + 2] = apus_swiglu_h(r.g[i].z, r.u[i].z, a.limit);
            v[4 * i + 3] = apus_swiglu_h(r.g[i].w, r.u[i].w, a.limit);
        }
    }
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) m = fmaxf(m, fabsf(v[i]));
    m = fmaxf(m, __shfl_xor(m, 1, 64));
    m = fmaxf(m, __shfl_xor(m, 2, 64));
    m = fmaxf(m, __shfl_xor(m, 4, 64));
    const uint32_t e = apus_act_scale_exp(m);
    const float inv = apus_inv_pow2_from_exp(e);
    uint32_t w4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        w4[i] = apus_e4m3_pack4_hw(v[4 * i] * inv, v[4 * i + 1] * inv, v[4 * i + 2] * inv,
                                   v[4 * i + 3] * inv);
    *reinterpret_cast<uint4 *>(lcodes + r.row * LDK + r.q * 128 + sub * 16) =
        uint4{w4[0], w4[1], w4[2], w4[3]};
    if (sub == 0) lsc[r.row * NQ + r.q] = (uint8_t)e;
}

/* the K-quarter-order instance at K = 2048 (the routed few-row w2) held to 4
 * waves per SIMD: 126 VGPRs, no spills (unconstrained 126 + 16 AGPRs, 3
 * waves); config 2 443-445 -> 434-441 us, the 64-token sublayer 456-461 ->
 * 446-454 us (same box, alternating) */
#ifndef APUS_DEC_FOLD_WPE
#define APUS_DEC_FOLD_WPE 4
#endif
template <int WF, int R, int NS, int PD, int KS, int ASRC, bool FOLD>
__global__ __launch_bounds__(APUS_DEC_NT)
__attribute__((amdgpu_waves_per_eu(FOLD && NS == 4 ? APUS_DEC_FOLD_WPE : 1))) void apus_gemm_decode_kernel(ApusGemmArgs args) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ int last_ticket;
    constexpr int K = NS * 512, NQ = NS * 4, K16 = K / 16, LDK = K + 32;
    constexpr int NSW = NS / KS;                       /* slices per wave */
    constexpr int TPW = APUS_DEC_WAVES / KS;           /* row tiles per workgroup */
    static_assert(NS % KS == 0 && PD <= NSW && APUS_DEC_WAVES % KS == 0, "decode shape");
    /* FOLD: the K-quarter order (four chains from zero over the quarters of
     * K, added left to right), with whole-K waves */
    static_assert(!FOLD || (KS == 1 && NS % 4 == 0), "K-quarter fold needs whole-K waves");
    constexpr int QS = NS / 4;                         /* slices per K quarter */
    if (args.zero && blockIdx.y == 0) {
        for (int i = blockIdx.x * APUS_DEC_NT + threadIdx.x; i < args.nzero; i += gridDim.x * APUS_DEC_NT)
            args.zero[i] = 0u;
    }
    /* quantising staging: when the first chunk's activation rows are known
     * without the entry (routed pair, single entry), their loads go out
     * before the entry lookup */
    ApusStageRaw<ASRC> raw0;
    bool pre = false;
    if constexpr (ASRC != APUS_A_CODES) {
        if (!args.ents && args.pidx) {
            apus_stage_load<K, ASRC>(args, nullptr, (blockIdx.y / args.nmat) / args.adiv, 0, 1, 0, raw0);
            pre = true;
        } else if (!args.ents) {
            apus_stage_load<K, ASRC>(args, args.ent0.arows, args.ent0.a0, 0, min(R, args.ent0.M), 0, raw0);
            pre = true;
        }
    }
    const ApusGemmEnt ent = apus_entry_of(args, blockIdx.y);
    const bool active = ent.M > args.m_min && !(args.m_max > 0 && ent.M > args.m_max);
    if (!active && !args.acc_y) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    /* KS waves share a row tile and split its K range */
    const int tile = blockIdx.x * TPW + wave / KS;
    const int kpart = wave % KS;
    const int o = tile * 16 + r;
    uint8_t *lcodes = lds;
    uint8_t *lsc = lds + R * LDK;
    apus_v4f *lred = reinterpret_cast<apus_v4f *>(lds + ((R * LDK + R * NQ + 15) & ~15));
    const ApusWLane wl = apus_wlane<WF>(ent, args.wtiled, o, lane, K);

    const int sbase = kpart * NSW;
    /* FP4: the group-scale bytes of every slice of this wave's stream, one
     * burst ahead of the weight ring (loaded with each slice instead, as
     * separate small loads into the scale array, the config-0 launch ran
     * ~0.3 us slower) */
    constexpr bool SCU = WF == APUS_W_FP4 && APUS_DEC_SC_UPFRONT;
    apus_v4u scs[SCU ? NSW : 1];
    if constexpr (SCU) {
#pragma unroll
        for (int si = 0; si < NSW; ++si) scs[si] = apus_gld<apus_v4u>(wl.s + (size_t)(sbase + si) * wl.ss);
    }
    for (int c0 = 0; active && c0 < ent.M; c0 += R) {
        const int rows = min(R, ent.M - c0);
        apus_lds_barrier();           /* the previous chunk's LDS reads are done */
        ApusBFrag<WF> ring[PD];
        if constexpr (ASRC == APUS_A_CODES) {
            /* weight prefetch ring first: the staging below waits on its
             * loads through branches (vmcnt 0), so issuing the ring after it
             * would start the weight stream one or two memory round trips
             * late (config-0 launch 11.25 -> 11.11 us with the ring first) */
#pragma unroll
            for (int u = 0; u < PD; ++u) apus_load_b_full<WF, !SCU>(ring[u], wl, sbase + u);
            /* stage: row indices, then every code/scale load, then the LDS
             * writes */
            int ridx[R];
            if (ent.arows) {
#pragma unroll
                for (int j = 0; j < R; ++j) ridx[j] = apus_gld<int>(ent.arows + (c0 + min(j, rows - 1)));
            } else {
#pragma unroll
                for (int j = 0; j < R; ++j) ridx[j] = ent.a0 + c0 + min(j, rows - 1);
            }
            /* a row is K16 16-byte pieces: RPJ rows per pass of the APUS_DEC_NT
             * threads when K16 <= APUS_DEC_NT, else CPR passes per row */
            constexpr int RPJ = K16 <= APUS_DEC_NT ? APUS_DEC_NT / K16 : 1;
            constexpr int CPR = K16 <= APUS_DEC_NT ? 1 : K16 / APUS_DEC_NT;
            constexpr int STAGE = K16 <= APUS_DEC_NT ? R * K16 / APUS_DEC_NT : R * CPR;
            static_assert(RPJ >= 1 && R % RPJ == 0 && (K16 <= APUS_DEC_NT || K16 % APUS_DEC_NT == 0), "staging shape");
            uint4 v[STAGE];
#pragma unroll
            for (int j = 0; j < STAGE; ++j) {
                int row, cc;
                if constexpr (K16 <= APUS_DEC_NT) {
                    const int rsub = threadIdx.x / K16;         /* 0..RPJ-1 */
                    row = j * RPJ + rsub;
                    cc = threadIdx.x - rsub * K16;
                } else {
                    row = j / CPR;
                    cc = (j % CPR) * APUS_DEC_NT + threadIdx.x;
                }
                int ar = ridx[0];
#pragma unroll
                for (int t = 1; t < R; ++t) ar = row == t ? ridx[t] : ar;
                /* unconditional: rows past the entry's read its last row
                 * again (ridx is clamped) and are not stored; a load behind
                 * a branch would make the compiler drain every load in
                 * flight, one memory round trip per row */
                v[j] = apus_ld16(args.acodes + (size_t)ar * K + cc * 16);
            }
            constexpr int SPT = (R * NQ + APUS_DEC_NT - 1) / APUS_DEC_NT;   /* scales per thread */
            float scv[SPT];
#pragma unroll
            for (int k = 0; k < SPT; ++k) {
                /* index clamped instead of a guarded load (no branch) */
                const int si = min(threadIdx.x + APUS_DEC_NT * k, R * NQ - 1), srr = si / NQ;
                int sar = ridx[0];
#pragma unroll
                for (int t = 1; t < R; ++t) sar = srr == t ? ridx[t] : sar;
                scv[k] = apus_gld<float>(args.ascale + ((size_t)sar * NQ + (si - srr * NQ)));
            }
#pragma unroll
            for (int j = 0; j < STAGE; ++j) {
                int row, cc;
                if constexpr (K16 <= APUS_DEC_NT) {
                    const int rsub = threadIdx.x / K16;
                    row = j * RPJ + rsub;
                    cc = threadIdx.x - rsub * K16;
                } else {
                    row = j / CPR;
                    cc = (j % CPR) * APUS_DEC_NT + threadIdx.x;
                }
                if (row < rows) *reinterpret_cast<uint4 *>(lcodes + row * LDK + cc * 16) = v[j];
            }
#pragma unroll
            for (int k = 0; k < SPT; ++k) {
                const int si = threadIdx.x + APUS_DEC_NT * k;
                if (si < R * NQ && si / NQ < rows) lsc[si] = (uint8_t)apus_e8m0_of(scv[k]);
            }
        } else {
            /* first pass: loads (unless issued before the entry lookup), the
             * weight ring, then the quantisation; later passes load and
             * quantise */
            ApusStageRaw<ASRC> r0;
            if (pre && c0 == 0) r0 = raw0;
            else apus_stage_load<K, ASRC>(args, ent.arows, ent.a0, c0, rows, 0, r0);
#pragma unroll
            for (int u = 0; u < PD; ++u) apus_load_b_full<WF, !SCU>(ring[u], wl, sbase + u);
            apus_stage_quant<K, ASRC>(args, r0, lcodes, lsc);
            constexpr int PASSES = (R * NQ + APUS_DEC_NT / 8 - 1) / (APUS_DEC_NT / 8);
#pragma unroll
            for (int pass = 1; pass < PASSES; ++pass) {
                ApusStageRaw<ASRC> rp;
                apus_stage_load<K, ASRC>(args, ent.arows, ent.a0, c0, rows, pass, rp);
                apus_stage_quant<K, ASRC>(args, rp, lcodes, lsc);
            }
        }
        apus_lds_barrier();
        const bool rvalid = r < rows;
        const int rr = rvalid ? r : 0;
        const uint8_t *arow = lcodes + rr * LDK + g * 16;
        const uint8_t *asrow = lsc + rr * NQ;
        const int z = rvalid ? -1 : 0;
        apus_v4f acc = {0.f, 0.f, 0.f, 0.f};
        apus_v4f tot = {-0.f, -0.f, -0.f, -0.f};      /* -0 + x == x for every x */
#pragma unroll
        for (int si = 0; si < NSW; ++si) {
            const int s = sbase + si;
            ApusBFrag<WF> &cur = ring[si % PD];
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const int q = s * 4 + st;
                const uint4 a0 = *reinterpret_cast<const uint4 *>(arow + q * 128);
                const uint4 a1 = *reinterpret_cast<const uint4 *>(arow + q * 128 + 64);
                const apus_v8i a = apus_v8i{(int)a0.x & z, (int)a0.y & z, (int)a0.z & z,
                                            (int)a0.w & z, (int)a1.x & z, (int)a1.y & z,
                                            (int)a1.z & z, (int)a1.w & z};
                const int sa = asrow[q];
                if constexpr (WF == APUS_W_FP4) {
                    const apus_v4u w = cur.w[st][0];
                    const apus_v8i b = apus_v8i{(int)w.x, (int)w.y, (int)w.z, (int)w.w, 0, 0, 0, 0};
                    const int sb = (int)(((SCU ? scs[SCU ? si : 0][st] : cur.s[st]) >> (8 * g)) & 0xffu);
                    acc = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E2M1, 0, 0>(a, b, acc, sa, sb);
                } else {
                    const apus_v4u w0 = cur.w[st][0], w1 = cur.w[st][1];
                    const apus_v8i b = apus_v8i{(int)w0.x, (int)w0.y, (int)w0.z, (int)w0.w,
                                                (int)w1.x, (int)w1.y, (int)w1.z, (int)w1.w};
                    acc = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E4M3, 0, 0>(a, b, acc, sa, (int)cur.s[st]);
                }
            }
            if (si + PD < NSW) apus_load_b_full<WF, !SCU>(cur, wl, s + PD);
            if constexpr (FOLD) {
                if ((si + 1) % QS == 0) {
                    tot += acc;
                    acc = apus_v4f{0.f, 0.f, 0.f, 0.f};
                }
            }
        }
        if constexpr (FOLD) acc = tot;
        if (KS > 1) {
            /* the K parts of a tile meet in LDS; part 0 adds them in part order */
            lred[wave * 64 + lane] = acc;
            __syncthreads();
            if (kpart == 0) {
#pragma unroll
                for (int p = 1; p < KS; ++p) acc += lred[(wave + p) * 64 + lane];
            }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int m = 4 * g + q;
            if (kpart == 0 && m < rows) {
                float val = acc[q];
                if (args.round_out) val = apus_bf16_rne(val);
                const int mm = c0 + m;
                const int orow = ent.orows ? apus_gld<int>(ent.orows + (mm)) : ent.o0 + mm;
                float *dst = ent.out + (size_t)orow * args.ldo + o;
                if (args.acc_y) /* device-coherent store: read by another workgroup */
                    __hip_atomic_store(dst, val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                else
                    apus_gst<float>(dst, val);
            }
        }
    }
    if (args.acc_y) {
        /* The outputs went out as device-coherent stores; once every wave
         * has seen them complete, take a ticket. The last workgroup of the
         * column tile reads every pair's outputs with device-coherent loads
         * (no stale copy in its own L2), so no cache-wide fence is needed. */
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (threadIdx.x == 0)
            last_ticket = __hip_atomic_fetch_add(&args.tickets[blockIdx.x], 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT) == gridDim.y - 1;
        __syncthreads();
        if (last_ticket) {
            constexpr int TW = 16 * TPW;
            const float *eo = args.pout[0];
            const int topk = args.acc_topk;
            for (int i = threadIdx.x; i < args.acc_s * TW; i += APUS_DEC_NT) {
                const int t = i / TW, oo = blockIdx.x * TW + (i - t * TW);
                float y = 0.0f;
                for (int j = 0; j < topk; ++j) {
                    const int pj = t * topk + j;
                    const float e = __hip_atomic_load(eo + (size_t)pj * args.ldo + oo, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT);
                    y = __fadd_rn(y, __fmul_rn(args.acc_w[pj], e));
                }
                args.acc_y[(size_t)t * args.ldo + oo] = y;
            }
        }
    }
}

/*
 * Prefill schedule (grouped launches whose entries have many rows, e.g.
 * routed experts over a 512-token prompt). A workgroup of 8 waves owns
 * 8 weight row tiles (128 rows) of one entry and takes the entry's rows in
 * chunks of TT token tiles (16*TT rows). For each 512-wide K slice the
 * chunk's activation codes are staged in LDS (double buffered: the loads of
 * slice s+1 are in flight while slice s is multiplied), and each wave
 * multiplies its weight fragment, held in a prefetch ring, against all TT
 * token tiles, so the weights are streamed from HBM once per chunk.
 * K = 512 * NS is a template constant (straight-line slice loop).
 */
#ifndef APUS_PRE_WAVES
#define APUS_PRE_WAVES 8
#endif
#define APUS_PRE_THREADS (64 * APUS_PRE_WAVES)

template <int WF, int NS, int TT, int PD, bool FOLD>
__global__ __launch_bounds__(APUS_PRE_THREADS, APUS_PRE_WAVES >= 16 ? 1 : 2) void apus_gemm_prefill_kernel(ApusGemmArgs args) {
    constexpr int K = NS * 512, NQ = NS * 4;
    /* FOLD: the K-quarter order (four chains from zero over the quarters of
     * K, added left to right) */
    static_assert(!FOLD || NS % 4 == 0, "K-quarter fold");
    constexpr int QS = NS / 4;
    constexpr int ROWS = 16 * TT;                 /* activation rows per chunk */
    constexpr int PITCH = 512 + 32;               /* LDS bytes per row per slice (measured best of 8..96 pad) */
    constexpr int CHUNKS = ROWS * 32 / APUS_PRE_THREADS;   /* 16-byte loads per thread per slice */
    static_assert(WF != APUS_W_FP4 || ROWS == APUS_PREFILL_ROWS, "work-list chunk");
    __shared__ __align__(16) uint8_t abuf[2][ROWS * PITCH];
    __shared__ uint8_t sbuf[2][ROWS * 4];
    /* launch row = entry, or one work-list item (entry, first row) */
    int eidx = blockIdx.y, cfirst = 0, cstep = ROWS;
    if (args.items) {
        const int2 it = apus_gld<int2>(args.items + blockIdx.y);
        if (it.x < 0) return;
        eidx = it.x; cfirst = it.y; cstep = 1 << 30;
    }
    const ApusGemmEnt ent = apus_gld<ApusGemmEnt>(args.ents + eidx);
    if (ent.M <= args.m_min || (args.m_max > 0 && ent.M > args.m_max)) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int o = (blockIdx.x * APUS_PRE_WAVES + wave) * 16 + r;   /* O % 128 == 0 */
    const ApusWLane wl = apus_wlane<WF>(ent, args.wtiled, o, lane, K);

    for (int c0 = cfirst; c0 < ent.M; c0 += cstep) {
        const int rows = min(ROWS, ent.M - c0);
        const int ntile = __builtin_amdgcn_readfirstlane((rows + 15) >> 4);
        /* the activation rows this thread stages (rows past the entry repeat
         * its last row; their outputs are never stored) */
        const uint8_t *abase[CHUNKS];
#pragma unroll
        for (int j = 0; j < CHUNKS; ++j) {
            const int i = threadIdx.x + j * APUS_PRE_THREADS;
            const int rr = min(i >> 5, rows - 1);
            const int ar = ent.arows ? apus_gld<int>(ent.arows + (c0 + rr)) : ent.a0 + c0 + rr;
            abase[j] = args.acodes + (size_t)ar * K + (i & 31) * 16;
        }
        const int srr = min((int)((threadIdx.x % (ROWS * 4)) >> 2), rows - 1);
        const int sar = ent.arows ? apus_gld<int>(ent.arows + (c0 + srr)) : ent.a0 + c0 + srr;
        const float *sbase = args.ascale + (size_t)sar * NQ + (threadIdx.x & 3);
        uint4 v[CHUNKS];
        float sv;
#define APUS_PRE_FETCH(S)                                                      \
        do {                                                                   \
            _Pragma("unroll") for (int j = 0; j < CHUNKS; ++j)                 \
                v[j] = apus_ld16(abase[j] + (S) * 512);                        \
            sv = sbase[(S) * 4];                                               \
        } while (0)
#define APUS_PRE_STORE(B)                                                      \
        do {                                                                   \
            _Pragma("unroll") for (int j = 0; j < CHUNKS; ++j) {               \
                const int i = threadIdx.x + j * APUS_PRE_THREADS;              \
                *reinterpret_cast<uint4 *>(&abuf[B][(i >> 5) * PITCH + (i & 31) * 16]) = v[j]; \
            }                                                                  \
            if (threadIdx.x < ROWS * 4) sbuf[B][threadIdx.x] = (uint8_t)apus_e8m0_of(sv); \
        } while (0)
        apus_lds_barrier();           /* previous chunk's readers are done */
        APUS_PRE_FETCH(0);
        APUS_PRE_STORE(0);
        apus_v4f acc[TT], tot[FOLD ? TT : 1];
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[t] = apus_v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < (FOLD ? TT : 1); ++t) tot[t] = apus_v4f{-0.f, -0.f, -0.f, -0.f};
        ApusBFrag<WF> ring[PD];
#pragma unroll
        for (int u = 0; u < PD; ++u) apus_load_b_full<WF>(ring[u], wl, u);
        apus_lds_barrier();
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            /* no instruction moves across slice boundaries: the unrolled
             * loop would otherwise hoist every slice's loads to the top */
            __builtin_amdgcn_sched_barrier(0);
            if (s + 1 < NS) APUS_PRE_FETCH(s + 1);
            ApusBFrag<WF> &cur = ring[s % PD];
            const uint8_t *ab = abuf[s & 1];
            const uint8_t *sb8 = sbuf[s & 1];
            {
                /* only the chunk's token tiles (a wave-uniform test); the
                 * rows of a partial last tile repeat the chunk's last row and
                 * their outputs are not stored */
#pragma unroll
                for (int t = 0; t < TT; ++t) {
                    if (t >= ntile) break;
                    const uint8_t *ap = ab + (t * 16 + r) * PITCH + g * 16;
#pragma unroll
                    for (int st = 0; st < 4; ++st) {
                        const uint4 a0 = *reinterpret_cast<const uint4 *>(ap + st * 128);
                        const uint4 a1 = *reinterpret_cast<const uint4 *>(ap + st * 128 + 64);
                        const apus_v8i a = apus_v8i{(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w,
                                                    (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
                        const int sa = sb8[(t * 16 + r) * 4 + st];
                        if (WF == APUS_W_FP4) {
                            const apus_v4u w = cur.w[st][0];
                            const apus_v8i b = apus_v8i{(int)w.x, (int)w.y, (int)w.z, (int)w.w, 0, 0, 0, 0};
                            const int sbv = (int)((cur.s[st] >> (8 * g)) & 0xffu);
                            acc[t] = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E2M1, 0, 0>(a, b, acc[t], sa, sbv);
                        } else {
                            const apus_v4u w0 = cur.w[st][0], w1 = cur.w[st][1];
                            const apus_v8i b = apus_v8i{(int)w0.x, (int)w0.y, (int)w0.z, (int)w0.w,
                                                        (int)w1.x, (int)w1.y, (int)w1.z, (int)w1.w};
                            acc[t] = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E4M3, 0, 0>(a, b, acc[t], sa, (int)cur.s[st]);
                        }
                    }
                    /* the tile's MFMAs complete here: MFMAs touch no memory,
                     * so the compiler would otherwise sink them all below
                     * the slice barriers and keep every operand live */
                    asm volatile("" : "+v"(acc[t]) :: "memory");
                }
            }
            if (s + PD < NS) apus_load_b_full<WF>(cur, wl, s + PD);
            if constexpr (FOLD) {
                if ((s + 1) % QS == 0) {
#pragma unroll
                    for (int t = 0; t < TT; ++t) {
                        tot[t] += acc[t];
                        acc[t] = apus_v4f{0.f, 0.f, 0.f, 0.f};
                    }
                }
            }
            if (s + 1 < NS) APUS_PRE_STORE((s + 1) & 1);
            apus_lds_barrier();
        }
        if constexpr (FOLD) {
#pragma unroll
            for (int t = 0; t < TT; ++t) acc[t] = tot[t];
        }
        {
#pragma unroll
            for (int t = 0; t < TT; ++t) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int m = t * 16 + 4 * g + q;
                    if (m < rows) {
                        float val = acc[t][q];
                        if (args.round_out) val = apus_bf16_rne(val);
                        const int mm = c0 + m;
                        const int orow = ent.orows ? apus_gld<int>(ent.orows + (mm)) : ent.o0 + mm;
                        apus_gst<float>(ent.out + ((size_t)orow * args.ldo + o), val);
                    }
                }
            }
        }
    }
}

/*
 * Prefill schedule with the activations resident in LDS (MXFP4 routed
 * experts over many-row work items: w1/w3 at K = 4096, w2 at K = 2048 in the
 * K-quarter order). A workgroup of 8 waves takes one work item (entry,
 * 64-row chunk), stages the chunk's activations for K [0, 2048) once (64
 * rows x 2048 codes, 130 KB of LDS), streams NCB consecutive 128-row column
 * blocks of the weight over that K range through one register ring that
 * runs across the blocks without a barrier (the activations are read-only
 * between stagings), and for K = 4096 then stages K [2048, 4096) and streams
 * the same blocks again, their accumulators kept in registers. Against
 * apus_gemm_prefill_kernel, whose workgroups restage the chunk for every
 * column block (as many activation bytes through L2 as weight bytes) and
 * meet at an LDS barrier every 512-slice, the L2 activation traffic drops
 * NCB-fold. Every output is the same chain (one over the 128-groups in
 * order, or four K-quarter chains added in order with FOLD), so the results
 * are bit-identical to it.
 */
#ifndef APUS_PRE_RA_NCB
#define APUS_PRE_RA_NCB 4
#endif
#ifndef APUS_PRE_RA_PD
#define APUS_PRE_RA_PD 2
#endif
template <int NS, bool FOLD, int NCB>
__global__ __launch_bounds__(512, 2) void apus_gemm_prefill_ra_kernel(ApusGemmArgs args) {
    constexpr int K = NS * 512, NQ = NS * 4, TT = 4, ROWS = 64, PD = APUS_PRE_RA_PD, NW = 8;
    constexpr int KP = 2048, NPH = K / KP, SPH = KP / 512;    /* staged K per phase, phases */
    constexpr int PITCH = KP + 32;                /* bytes per staged row (bank spread) */
    constexpr int LOADS = ROWS * (KP / 16) / (64 * NW);       /* 16-byte staging loads per thread */
    constexpr int SCL = ROWS * NQ / (64 * NW);                /* scale loads per thread */
    constexpr int STEPS = NPH * NCB * SPH;                    /* ring steps (512-slices) */
    static_assert(K % KP == 0 && (!FOLD || NS == 4) && ROWS * NQ % (64 * NW) == 0, "ra shape");
    extern __shared__ __align__(16) uint8_t ra_lds[];
    uint8_t *la = ra_lds;                          /* [ROWS][PITCH] codes of the phase */
    uint8_t *lsa = ra_lds + ROWS * PITCH;          /* [ROWS][NQ] E8M0 bytes */
    const int2 it = apus_gld<int2>(args.items + blockIdx.y);
    if (it.x < 0) return;
    const ApusGemmEnt ent = apus_gld<ApusGemmEnt>(args.ents + it.x);
    if (ent.M <= args.m_min || (args.m_max > 0 && ent.M > args.m_max)) return;
    const int c0 = it.y;
    const int rows = min(ROWS, ent.M - c0);
    const int ntile = __builtin_amdgcn_readfirstlane((rows + 15) >> 4);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    auto wlane = [&](int cb) {
        return apus_wlane<APUS_W_FP4>(ent, args.wtiled, ((blockIdx.x * NCB + cb) * NW + wave) * 16 + r, lane, K);
    };
    /* ring step k: phase k / (NCB SPH), block (k / SPH) % NCB, K slice
     * phase * SPH + k % SPH */
    auto slice_of = [](int k) { return (k / (NCB * SPH)) * SPH + k % SPH; };
    /* the weight ring first (block 0, the first slices) */
    ApusBFrag<APUS_W_FP4> ring[PD];
    ApusWLane wln = wlane(0);                      /* stream of the ring's next refill */
#pragma unroll
    for (int u = 0; u < PD; ++u) apus_load_b_full<APUS_W_FP4>(ring[u], wln, slice_of(u));
    /* activation row of each staging load and scale load (rows past the
     * chunk repeat its last row); thread t takes 16-byte piece (t + 512 j) %
     * 128 of row (t + 512 j) / 128 */
    int arow[LOADS];
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
        const int rr = min((threadIdx.x + j * 64 * NW) >> 7, rows - 1);
        arow[j] = ent.arows ? apus_gld<int>(ent.arows + (c0 + rr)) : ent.a0 + c0 + rr;
    }
    auto stage = [&](int ph) {
        uint4 v[LOADS];
#pragma unroll
        for (int j = 0; j < LOADS; ++j)
            v[j] = apus_ld16(args.acodes + (size_t)arow[j] * K + ph * KP + ((threadIdx.x + j * 64 * NW) & 127) * 16);
#pragma unroll
        for (int j = 0; j < LOADS; ++j) {
            const int i = threadIdx.x + j * 64 * NW;
            *reinterpret_cast<uint4 *>(la + (i >> 7) * PITCH + (i & 127) * 16) = v[j];
        }
    };
    stage(0);
    {
        float sv[SCL];
#pragma unroll
        for (int j = 0; j < SCL; ++j) {
            const int i = threadIdx.x + j * 64 * NW;   /* (row, group) = (i / NQ, i % NQ) */
            const int rr = min(i / NQ, rows - 1);
            const int ar = ent.arows ? apus_gld<int>(ent.arows + (c0 + rr)) : ent.a0 + c0 + rr;
            sv[j] = apus_gld<float>(args.ascale + (size_t)ar * NQ + (i % NQ));
        }
#pragma unroll
        for (int j = 0; j < SCL; ++j) lsa[threadIdx.x + j * 64 * NW] = (uint8_t)apus_e8m0_of(sv[j]);
    }
    /* the output rows of this lane's accumulator elements (looked up once:
     * a lookup behind the store's branch would drain the ring) */
    int orow[TT][4];
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int mm = c0 + min(t * 16 + 4 * g + q, rows - 1);
            orow[t][q] = ent.orows ? apus_gld<int>(ent.orows + mm) : ent.o0 + mm;
        }
    apus_lds_barrier();

    /* accumulators of the column blocks (kept across the phases; with one
     * phase a block's are stored right after it, so only one block's are
     * live at a time) */
    apus_v4f acc[NCB][TT], tot[FOLD ? NCB : 1][TT];
    auto store_block = [&](int cb) {
        const int o = ((blockIdx.x * NCB + cb) * NW + wave) * 16 + r;
#pragma unroll
        for (int t = 0; t < TT; ++t) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (t * 16 + 4 * g + q < rows) {
                    float val = FOLD ? tot[FOLD ? cb : 0][t][q] : acc[cb][t][q];
                    if (args.round_out) val = apus_bf16_rne(val);
                    apus_gst<float>(ent.out + ((size_t)orow[t][q] * args.ldo + o), val);
                }
            }
        }
    };
#pragma unroll
    for (int ph = 0; ph < NPH; ++ph) {
        if (ph > 0) {
            apus_lds_barrier();                    /* every wave is done with the phase before */
            stage(ph);
            apus_lds_barrier();
        }
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) {
            if (ph == 0) {
#pragma unroll
                for (int t = 0; t < TT; ++t) {
                    acc[cb][t] = apus_v4f{0.f, 0.f, 0.f, 0.f};
                    if constexpr (FOLD) tot[cb][t] = apus_v4f{-0.f, -0.f, -0.f, -0.f};
                }
            }
#pragma unroll
            for (int s = 0; s < SPH; ++s) {
                const int k = (ph * NCB + cb) * SPH + s;
                ApusBFrag<APUS_W_FP4> &cur = ring[k % PD];
#pragma unroll
                for (int t = 0; t < TT; ++t) {
                    if (t >= ntile) break;
                    const uint8_t *ap = la + (t * 16 + r) * PITCH + g * 16;
#pragma unroll
                    for (int st = 0; st < 4; ++st) {
                        const int ql = s * 4 + st, q = ph * SPH * 4 + ql;
                        const uint4 a0 = *reinterpret_cast<const uint4 *>(ap + ql * 128);
                        const uint4 a1 = *reinterpret_cast<const uint4 *>(ap + ql * 128 + 64);
                        const apus_v8i a = apus_v8i{(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w,
                                                    (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
                        const int sa = lsa[(t * 16 + r) * NQ + q];
                        const apus_v4u w = cur.w[st][0];
                        const apus_v8i b = apus_v8i{(int)w.x, (int)w.y, (int)w.z, (int)w.w, 0, 0, 0, 0};
                        const int sbv = (int)((cur.s[st] >> (8 * g)) & 0xffu);
                        acc[cb][t] = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E2M1, 0, 0>(a, b, acc[cb][t], sa, sbv);
                    }
                    /* keep the tile's MFMAs here (they touch no memory) */
                    asm volatile("" : "+v"(acc[cb][t]) :: "memory");
                }
                /* refill: step k + PD, possibly in the next block or phase */
                if (k + PD < STEPS) {
                    const int kn = k + PD;
                    if (kn % SPH == 0) wln = wlane((kn / SPH) % NCB);
                    apus_load_b_full<APUS_W_FP4>(cur, wln, slice_of(kn));
                }
                if constexpr (FOLD) {
                    /* the K-quarter order: one chain per 512-slice, added in order */
#pragma unroll
                    for (int t = 0; t < TT; ++t) {
                        tot[cb][t] += acc[cb][t];
                        acc[cb][t] = apus_v4f{0.f, 0.f, 0.f, 0.f};
                    }
                }
            }
            if (NPH == 1) store_block(cb);
        }
    }
    if (NPH > 1) {
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) store_block(cb);
    }
}

/* launch the resident-activation schedule (returns false where it does not
 * apply) */
template <int NS, bool FOLD>
bool apus_launch_pre_ra(const ApusGemmArgs &p, int n_ent, hipStream_t st) {
    constexpr size_t lds = 64 * (2048 + 32) + 64 * (NS * 4);
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void *>(&apus_gemm_prefill_ra_kernel<NS, FOLD, APUS_PRE_RA_NCB>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (attr != hipSuccess) return false;
    dim3 gr(p.O / (128 * APUS_PRE_RA_NCB), n_ent);
    hipLaunchKernelGGL((apus_gemm_prefill_ra_kernel<NS, FOLD, APUS_PRE_RA_NCB>), gr, dim3(512), lds, st, p);
    return true;
}

/*
 * Tile schedule (dense GEMMs with more than 8 rows, e.g. a 512-token FP8
 * projection). A workgroup computes 64 rows (tokens) x 128 columns (weight
 * rows) over the whole K, one accumulation chain per output in 128-group
 * order. NW waves own TM x TN MFMA tiles each, all 64 tokens per wave (each
 * weight fragment loaded by one wave only): 4 waves of 64 x 32 weight rows
 * for K >= 4096, 8 waves of 64 x 16 for K <= 2048. Measured on gfx950: M =
 * 512, K = N = 4096: 4 waves of 32 tokens x 64 rows 22.7 us, of 64 x 32
 * 22.0 us, 8 waves of 64 x 16 22.5 us; K = 2048 (64 tokens): 4 waves 28.1
 * us, 8 waves 24.3 us. The 64 activation
 * rows of each group are staged in LDS (double buffered, loaded DA groups
 * ahead through a register ring); each wave streams its weight fragments straight into a register
 * ring PD groups ahead. The activation loads of a step are issued before
 * that step's weight loads, so waiting for them never waits for the ring.
 * K = 128 * NQ is a template constant (the group loop is straight-line).
 */
template <int WF, int TN>
struct ApusTileB {
    apus_v4u w[TN][WF == APUS_W_FP4 ? 1 : 2];
    unsigned s[TN];          /* FP4: the row's 4 group-scale bytes of this step */
};

/* NW waves; TM: 16-token fragments per wave, so 4 / TM waves along the
 * tokens and NW * TM / 4 along the weight rows, each owning TN 16-row tiles */
template <int WF, int NQ, int PD, int DA, int TM, int NW>
__global__ __launch_bounds__(64 * NW) void apus_gemm_tile_kernel(ApusGemmArgs args) {
    constexpr int WMW = 4 / TM;                /* waves along tokens */
    constexpr int WNW = NW / WMW;              /* waves along weight rows */
    constexpr int TN = 8 / WNW;                /* weight tiles per wave */
    constexpr int SP = NW;                     /* staging threads per token row */
    constexpr int SB = 128 / SP;               /* staged bytes per thread per group */
    static_assert(WMW * TM == 4 && WNW * TN == 8 && SB % 16 == 0, "tile shape");
    constexpr int BM = 64, BN = 128, LDA = 128 + 16;
    constexpr int K = NQ * 128;
    constexpr size_t RB = WF == APUS_W_FP4 ? K / 2 : K;     /* weight row bytes */
    /* FP: three LDS stages, and each step reads the next step's activation
     * fragments into registers before its own MFMAs, so LDS latency hides
     * behind the matrix cores instead of following the barrier */
    constexpr bool FP = APUS_TILE_FP != 0;
    constexpr int NB = FP ? 3 : 2;
    __shared__ __align__(16) uint8_t la[NB][BM * LDA];
    __shared__ uint8_t lsa[NB][BM];
    const ApusGemmEnt ent = args.ents ? apus_gld<ApusGemmEnt>(args.ents + blockIdx.z) : args.ent0;
    const int m0 = blockIdx.y * BM;
    if (m0 >= ent.M) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int wm = wave / WNW, wn = wave % WNW;
    const int nbase = blockIdx.x * BN + wn * (16 * TN);
    /* activation staging: thread t loads bytes [(t%SP)*SB, +SB) of token row t/SP */
    const int srow = threadIdx.x / SP, spart = threadIdx.x % SP;
    const int sm = m0 + srow;
    const int sar = sm < ent.M ? (ent.arows ? apus_gld<int>(ent.arows + sm) : ent.a0 + sm)
                               : (ent.arows ? apus_gld<int>(ent.arows) : ent.a0);
    const uint8_t *sap = args.acodes + (size_t)sar * K + spart * SB;
    const float *ssp = args.ascale + (size_t)sar * NQ;
    /* lane stream of the first of the wave's four 16-row tiles; the others
     * follow at tstride (weights) and sstride (FP4 scales) */
    const bool tiled = args.wtiled;
    const ApusWLane wl = apus_wlane<WF>(ent, tiled, nbase + r, lane, K);
    const size_t tstride = tiled ? (size_t)NQ * 16 * 64 * (WF == APUS_W_FP4 ? 1 : 2) : 16 * RB;
    const size_t sstride = tiled ? (size_t)(K / 512) * 256 : 16 * (K / 32);
    const uint8_t *wsrow = ent.ws + (size_t)blockIdx.x * NQ;     /* FP8 tile scales */
    /* FP8: the 128 x 128 tile scales of this column block, all groups */
    unsigned sb8[WF == APUS_W_FP8 ? NQ / 4 : 1];
    if constexpr (WF == APUS_W_FP8) {
#pragma unroll
        for (int i = 0; i < NQ / 4; ++i) sb8[i] = apus_gld<unsigned>(wsrow + 4 * i);
    }
    auto load_b = [&](ApusTileB<WF, TN> &f, int q) {
#pragma unroll
        for (int i = 0; i < TN; ++i) {
            const uint8_t *p = wl.w + i * tstride + (size_t)q * wl.qs;
            if constexpr (WF == APUS_W_FP4) {
                f.w[i][0] = apus_gld<apus_v4u>(p);
                f.s[i] = apus_gld<unsigned>(wl.s + i * sstride + (q >> 2) * wl.ss + (q & 3) * 4);
            } else {
                f.w[i][0] = apus_gld<apus_v4u>(p);
                f.w[i][1] = apus_gld<apus_v4u>(p + (wl.qs >> 1));
            }
        }
    };
    uint4 areg[DA][SB / 16];  /* activation ring: DA groups ahead */
    float sreg[DA];
    auto load_a = [&](int q, int slot) {
#pragma unroll
        for (int i = 0; i < SB / 16; ++i) areg[slot][i] = apus_ld16(sap + q * 128 + 16 * i);
        sreg[slot] = apus_gld<float>(ssp + q);    /* unconditional: no branch around a load */
    };
    auto store_a = [&](int q, int slot) {
        uint8_t *d = la[q % NB] + srow * LDA + spart * SB;
#pragma unroll
        for (int i = 0; i < SB / 16; ++i) *reinterpret_cast<uint4 *>(d + 16 * i) = areg[slot][i];
        if (spart == 0) lsa[q % NB][srow] = (uint8_t)apus_e8m0_of(sreg[slot]);
    };

    ApusTileB<WF, TN> ring[PD];
#pragma unroll
    for (int u = 0; u < DA; ++u)
        if (u < NQ) load_a(u, u);
#pragma unroll
    for (int u = 0; u < PD; ++u) load_b(ring[u], u);
    store_a(0, 0);
    if constexpr (FP) {
        static_assert(!FP || DA >= 2, "two staged groups ahead");
        if (NQ > 1) store_a(1, 1);
    }
    apus_lds_barrier();

    apus_v4f acc[TM][TN];
#pragma unroll
    for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int i = 0; i < TN; ++i) acc[t][i] = apus_v4f{0.f, 0.f, 0.f, 0.f};

    /* activation fragments of step q: rows wm*32 + 16t + r */
    struct Frag { apus_v8i a[TM]; int sa[TM]; };
    auto read_frag = [&](Frag &f, int q) {
        const uint8_t *ab = la[q % NB];
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            const int row = wm * 32 + t * 16 + r;
            const uint4 a0 = *reinterpret_cast<const uint4 *>(ab + row * LDA + g * 16);
            const uint4 a1 = *reinterpret_cast<const uint4 *>(ab + row * LDA + 64 + g * 16);
            f.a[t] = apus_v8i{(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w,
                              (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
            f.sa[t] = lsa[q % NB][row];
        }
    };
    if constexpr (FP) {
        Frag fc, fn;
        read_frag(fc, 0);
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            /* activation rows of step q + DA (slot of step q, staged two steps ago) */
            if (q + DA < NQ) load_a(q + DA, q % DA);
            if (q + 1 < NQ) read_frag(fn, q + 1);
            ApusTileB<WF, TN> &cur = ring[q % PD];
#pragma unroll
            for (int t = 0; t < TM; ++t) {
#pragma unroll
                for (int i = 0; i < TN; ++i) {
                    if constexpr (WF == APUS_W_FP4) {
                        const apus_v4u w = cur.w[i][0];
                        const apus_v8i b = apus_v8i{(int)w.x, (int)w.y, (int)w.z, (int)w.w, 0, 0, 0, 0};
                        const int sb = (int)((cur.s[i] >> (8 * g)) & 0xffu);
                        acc[t][i] = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E2M1, 0, 0>(fc.a[t], b, acc[t][i],
                                                                                         fc.sa[t], sb);
                    } else {
                        const apus_v4u w0 = cur.w[i][0], w1 = cur.w[i][1];
                        const apus_v8i b = apus_v8i{(int)w0.x, (int)w0.y, (int)w0.z, (int)w0.w,
                                                    (int)w1.x, (int)w1.y, (int)w1.z, (int)w1.w};
                        const int sb = (int)((sb8[q >> 2] >> (8 * (q & 3))) & 0xffu);
                        acc[t][i] = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E4M3, 0, 0>(fc.a[t], b, acc[t][i],
                                                                                         fc.sa[t], sb);
                    }
                }
            }
            if (q + PD < NQ) load_b(cur, q + PD);
            if (q + 2 < NQ) store_a(q + 2, (q + 2) % DA);
            apus_lds_barrier();
            fc = fn;
        }
    } else
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        /* activation rows of step q + DA (slot of step q, written last step) */
        if (q + DA < NQ) load_a(q + DA, q % DA);
        ApusTileB<WF, TN> &cur = ring[q % PD];
        const uint8_t *ab = la[q % NB];
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            const int row = wm * 32 + t * 16 + r;
            const uint4 a0 = *reinterpret_cast<const uint4 *>(ab + row * LDA + g * 16);
            const uint4 a1 = *reinterpret_cast<const uint4 *>(ab + row * LDA + 64 + g * 16);
            const apus_v8i a = apus_v8i{(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w,
                                        (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
            const int sa = lsa[q % NB][row];
#pragma unroll
            for (int i = 0; i < TN; ++i) {
                if constexpr (WF == APUS_W_FP4) {
                    const apus_v4u w = cur.w[i][0];
                    const apus_v8i b = apus_v8i{(int)w.x, (int)w.y, (int)w.z, (int)w.w, 0, 0, 0, 0};
                    const int sb = (int)((cur.s[i] >> (8 * g)) & 0xffu);
                    acc[t][i] = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E2M1, 0, 0>(a, b, acc[t][i], sa, sb);
                } else {
                    const apus_v4u w0 = cur.w[i][0], w1 = cur.w[i][1];
                    const apus_v8i b = apus_v8i{(int)w0.x, (int)w0.y, (int)w0.z, (int)w0.w,
                                                (int)w1.x, (int)w1.y, (int)w1.z, (int)w1.w};
                    const int sb = (int)((sb8[q >> 2] >> (8 * (q & 3))) & 0xffu);
                    acc[t][i] = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E4M3, 0, 0>(a, b, acc[t][i], sa, sb);
                }
            }
        }
        if (q + PD < NQ) load_b(cur, q + PD);
        if (q + 1 < NQ) store_a(q + 1, (q + 1) % DA);
        apus_lds_barrier();
    }
    /* lane holds D[4g + j][r]: token m0 + 32 wm + 16 t + 4g + j, weight row nbase + 16 i + r.
     * Without a row table the stores go out back to back; a row lookup
     * between stores waits (vmcnt, which on gfx9 also counts stores) for
     * every store before it (config 1, M = 512: 21.7 -> 20.5 us) */
    auto store_row = [&](float *dst, int t, int j) {
#pragma unroll
        for (int i = 0; i < TN; ++i) {
            float v = acc[t][i][j];
            if (args.round_out) v = apus_bf16_rne(v);
            apus_gst<float>(dst + i * 16, v);
        }
    };
    if (!ent.orows) {
#pragma unroll
        for (int t = 0; t < TM; ++t)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int mm = m0 + wm * 32 + t * 16 + 4 * g + j;
                if (mm < ent.M) store_row(ent.out + (size_t)(ent.o0 + mm) * args.ldo + nbase + r, t, j);
            }
    } else {
#pragma unroll
        for (int t = 0; t < TM; ++t)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int mm = m0 + wm * 32 + t * 16 + 4 * g + j;
                if (mm < ent.M)
                    store_row(ent.out + (size_t)apus_gld<int>(ent.orows + mm) * args.ldo + nbase + r, t, j);
            }
    }
}

/*
 * LDS tile schedule for dense FP8 GEMMs with more than 8 rows on MFMA-tiled
 * weights (e.g. a 512-token projection): the same 64 x 128 output tile and
 * the same accumulation chain per output (one chain over the 128-groups in
 * order) as apus_gemm_tile_kernel, so the two give identical bits, but both
 * operands travel global -> LDS directly (global_load_lds_dwordx4, no
 * register staging) through NST stages of one 128-group each, read by 8
 * waves (4 x 2, each 16 tokens x 64 weight rows). Per stage: 8 loads of 8
 * whole activation rows (each row's 16-byte chunks XOR-swizzled by the row
 * so the fragment reads are conflict-free) and 16 loads of 1 KB weight
 * fragments (the tiled layout is the MFMA operand order), 3 per wave; the
 * activation scales of every group go to LDS once, up front. Workgroup b
 * takes tile (b & 7) * (tiles / 8) + (b >> 3) when tiles % 8 == 0, so each
 * XCD (workgroups are dealt to the 8 XCDs round robin) works on one band of
 * weight-row blocks and every token block: its weight bytes come from HBM
 * once into that XCD's L2. Measured on gfx950 at M = 512, O = K = 4096 (a
 * fresh weight copy per launch): 17.7 us against 20.6 us for the register-
 * ring tile schedule; 3 / 4 / 5 stages 18.1 / 17.7 / 18.0 us; staging the
 * output through LDS for whole-row stores 18.1; 256 x 128 tiles split over
 * K in 2 or 4 (partners on one XCD, partial sums through L2) 20.9-25.5 us:
 * the partial sums' traffic costs more than the operand bytes they save.
 */
#define APUS_LT_NST 4
#ifndef APUS_PRE_LDS_NST
#define APUS_PRE_LDS_NST 3
#endif
typedef __attribute__((address_space(3))) void apus_lds_void;
typedef const __attribute__((address_space(1))) void apus_gbl_void;
/* 16 (or 4) bytes per lane from global memory straight into LDS at
 * lds + 16 * lane (4 * lane); lds must be the same in every lane */
__device__ __forceinline__ void apus_g2lds16(const void *g, unsigned lds) {
    __builtin_amdgcn_global_load_lds((apus_gbl_void *)g,
                                     (apus_lds_void *)(uintptr_t)__builtin_amdgcn_readfirstlane(lds), 16, 0, 0);
}
__device__ __forceinline__ void apus_g2lds4(const void *g, unsigned lds) {
    __builtin_amdgcn_global_load_lds((apus_gbl_void *)g,
                                     (apus_lds_void *)(uintptr_t)__builtin_amdgcn_readfirstlane(lds), 4, 0, 0);
}
template <int N>
__device__ __forceinline__ void apus_wait_vm() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

template <int NQ>
__global__ __launch_bounds__(512, 1) void apus_gemm_lds_kernel(ApusGemmArgs args) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int NST = APUS_LT_NST < NQ ? APUS_LT_NST : NQ;
    constexpr int K = NQ * 128;
    constexpr int BM = 64, AB = BM * 128, STB = AB + 128 * 128;
    constexpr int LA = BM / 8, LPW = (LA + 16) / 8;
    constexpr int SI = NQ;                     /* scale loads: one per group (64 rows) */
    static_assert(SI % 8 == 0, "scale loads");
    const ApusGemmEnt ent = args.ent0;
    float *lsc = reinterpret_cast<float *>(lds + NST * STB);     /* [q][64 rows] fp32 */
    const int M = ent.M;
    const int MT = (M + BM - 1) / BM, tiles = MT * (args.O >> 7);
    const int b = blockIdx.x;
    const int t = (tiles & 7) == 0 ? (b & 7) * (tiles >> 3) + (b >> 3) : b;
    const int mb = t % MT, nb = t / MT;
    const int m0 = mb * BM, n0 = nb * 128;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int wm = wave >> 1, wn = wave & 1;
    const unsigned lbase = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds);
    /* this wave's loads of a stage: activation instructions ii < LA (8 rows
     * each: lane -> row 8 ii + lane / 8, LDS slot lane % 8 holding 16-byte
     * chunk (lane % 8) ^ swizzle(row)), then weight fragments */
    const uint8_t *src[LPW];
    unsigned dst[LPW], qs[LPW];
#pragma unroll
    for (int u = 0; u < LPW; ++u) {
        const int ii = wave * LPW + u;
        if (ii < LA) {
            const int lr = 8 * ii + (lane >> 3), p = lane & 7;
            const int row = ent.a0 + (m0 + lr < M ? m0 + lr : M - 1);
            const int sw = apus_row_swz(lr);
            src[u] = args.acodes + (size_t)row * K + (p ^ sw) * 16;
            dst[u] = ii * 1024;
            qs[u] = 128;
        } else {
            const int f = (ii - LA) >> 1, h = (ii - LA) & 1;
            src[u] = ent.w + ((size_t)((n0 >> 4) + f) * NQ) * 2048 + h * 1024 + lane * 16;
            dst[u] = AB + f * 2048 + h * 1024;
            qs[u] = 2048;
        }
    }
    auto issue = [&](int q, int slot) {
#pragma unroll
        for (int u = 0; u < LPW; ++u) apus_g2lds16(src[u] + q * qs[u], lbase + slot * STB + dst[u]);
    };
#pragma unroll
    for (int u = 0; u < SI / 8; ++u) {
        const int q = wave * (SI / 8) + u;
        const int row = ent.a0 + (m0 + lane < M ? m0 + lane : M - 1);
        apus_g2lds4(args.ascale + (size_t)row * NQ + q, lbase + NST * STB + q * BM * 4);
    }
#pragma unroll
    for (int st = 0; st < NST; ++st) issue(st, st);
    const uint8_t *wsp = ent.ws + (size_t)nb * NQ;     /* 128 x 128 tile scales of this block */
    unsigned sbw[NQ / 4];
#pragma unroll
    for (int i = 0; i < NQ / 4; ++i) sbw[i] = __builtin_amdgcn_readfirstlane(apus_gld<unsigned>(wsp + 4 * i));

    apus_v4f acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = apus_v4f{0.f, 0.f, 0.f, 0.f};
    struct Frag { apus_v8i a, b[4]; int sa; };
    const int arow = wm * 16 + r;
    const int sw = apus_row_swz(r);
    auto read_frag = [&](Frag &f, int q) {
        const uint8_t *stg = lds + (q % NST) * STB;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint8_t *p = stg + AB + (wn * 4 + i) * 2048 + lane * 16;
            const apus_v4u lo = *reinterpret_cast<const apus_v4u *>(p);
            const apus_v4u hi = *reinterpret_cast<const apus_v4u *>(p + 1024);
            f.b[i] = apus_v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        }
        const uint8_t *p = stg + arow * 128;
        const apus_v4u lo = *reinterpret_cast<const apus_v4u *>(p + ((g ^ sw) << 4));
        const apus_v4u hi = *reinterpret_cast<const apus_v4u *>(p + (((4 + g) ^ sw) << 4));
        f.a = apus_v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        f.sa = (int)apus_e8m0_of(lsc[q * BM + arow]);
    };
    /* stage q is in LDS once at most (stages issued after it) x LPW loads
     * are in flight: NST - 1 stages follow stage 0 before the loop; in the
     * loop stage_ready(q) runs before stage q + NST - 1 is issued */
    auto stage_ready = [&](int q) {
        const int last = q == 0 ? NST - 1 : (q + NST - 2 < NQ - 1 ? q + NST - 2 : NQ - 1);
        const int ahead = last - q;
        if (ahead >= 3) apus_wait_vm<3 * LPW>();
        else if (ahead == 2) apus_wait_vm<2 * LPW>();
        else if (ahead == 1) apus_wait_vm<LPW>();
        else apus_wait_vm<0>();
        apus_lds_barrier();
    };
    static_assert(NST <= 4, "stage_ready waits for at most 3 stages ahead");
    Frag fr[2];
    stage_ready(0);
    read_frag(fr[0], 0);
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        if (q + 1 < NQ) {
            stage_ready(q + 1);
            if (q + NST < NQ) issue(q + NST, (q + NST) % NST);
            read_frag(fr[(q + 1) & 1], q + 1);
        }
        const Frag &f = fr[q & 1];
        const int sbq = (int)((sbw[q >> 2] >> (8 * (q & 3))) & 0xffu);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            acc[i] = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E4M3, 0, 0>(f.a, f.b[i], acc[i], f.sa, sbq);
    }
    /* lane holds D[4g + j][r]: token m0 + 16 wm + 4 g + j, weight row n0 + 64 wn + 16 i + r */
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int mm = m0 + wm * 16 + 4 * g + j;
        if (mm < M) {
            float *d = ent.out + (size_t)(ent.o0 + mm) * args.ldo + n0 + wn * 64 + r;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float v = acc[i][j];
                if (args.round_out) v = apus_bf16_rne(v);
                apus_gst<float>(d + i * 16, v);
            }
        }
    }
}

/*
 * Narrow schedule for dense FP8 GEMMs with 9..64 rows on tiled weights
 * (batched decode: a projection of 16-64 tokens). The tile schedules give
 * such a launch only O / 128 workgroups (32 for a 4096-row weight), each
 * streaming 512 KB: 14-17 us where M = 1 takes 6.5. Here a workgroup owns one
 * 16-row weight tile and all M rows (TM 16-row token tiles), and its 4 waves
 * split K in four contiguous quarters (every fragment then has exactly one
 * reader). Each wave streams its weight fragments into a register ring and
 * its activation rows global -> LDS into a wave-private ring (8 whole
 * 128-byte rows per load, 16-byte chunks XOR-swizzled by row for
 * conflict-free fragment reads; activation fragments loaded straight into
 * registers instead measured 6.2 / 12.3 us at M = 16 / 64), PD = 4 groups
 * ahead (3: 6.2 / 10.8, 2: 6.6 / 11.0). The four partial sums meet in LDS
 * and are added in K order.
 * Measured at O = K = 4096 (fresh weight copy per launch): M = 16 5.9 us,
 * M = 64 10.4 us, against 14.0 / 16.7 on the tile schedules; 8 waves splitting
 * K 12.9-13.0 at M = 64, 2 waves 13.1, two weight tiles per workgroup
 * 16.0, four 23.5, whole-K single-wave workgroups 80 (all before the LDS
 * activation ring).
 */
template <int NQ, int TM, int PDM, bool AL>
__global__ __launch_bounds__(256) void apus_gemm_narrow_kernel(ApusGemmArgs args) {
    constexpr int K = NQ * 128, NG = NQ / 4, PD = NG < PDM ? NG : PDM;
    constexpr int NL = 2 + 3 * TM;                   /* vector loads per group */
    constexpr int SLOT = TM * 2048;                  /* activation bytes per group */
    __shared__ apus_v4f red[4][TM][64];
    extern __shared__ __align__(16) uint8_t lring[];    /* AL: 4 waves x PD x SLOT */
    const ApusGemmEnt ent = args.ent0;
    const int M = ent.M;
    const int tile = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int q0 = wave * NG;
    const uint8_t *ap[TM], *lp[2 * TM];
    const float *sp[TM];
#pragma unroll
    for (int t = 0; t < TM; ++t) {
        const int row = ent.a0 + (16 * t + r < M ? 16 * t + r : M - 1);
        ap[t] = args.acodes + (size_t)row * K + g * 16;
        sp[t] = args.ascale + (size_t)row * NQ;
        /* LDS loads: instruction (t, hh) brings rows 16 t + 8 hh + lane / 8 */
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int lr = 8 * hh + (lane >> 3);
            const int rw = ent.a0 + (16 * t + lr < M ? 16 * t + lr : M - 1);
            const int sw = apus_row_swz(lr);
            lp[2 * t + hh] = args.acodes + (size_t)rw * K + ((lane & 7) ^ sw) * 16;
        }
    }
    uint8_t *wring = lring + (AL ? wave * PD * SLOT : 0);
    const unsigned wbase = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)wring);
    const uint8_t *bp = ent.w + ((size_t)tile * NQ * 128 + lane) * 16;
    const uint8_t *wsp = ent.ws + (size_t)(tile >> 3) * NQ + q0;     /* 128 x 128 tile scales */
    unsigned sbw[(NG + 3) / 4];
#pragma unroll
    for (int i = 0; i < (NG + 3) / 4; ++i)
        sbw[i] = __builtin_amdgcn_readfirstlane(apus_gld<unsigned>(wsp + 4 * i));
    struct Grp { apus_v4u b0, b1, a0[AL ? 1 : TM], a1[AL ? 1 : TM]; float s[TM]; };
    auto load = [&](Grp &f, int i) {
        const int q = q0 + i;
        f.b0 = apus_ld16_stream(bp + (size_t)q * 2048);
        f.b1 = apus_ld16_stream(bp + (size_t)q * 2048 + 1024);
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            if constexpr (AL) {
                apus_g2lds16(lp[2 * t] + q * 128, wbase + (i % PD) * SLOT + t * 2048);
                apus_g2lds16(lp[2 * t + 1] + q * 128, wbase + (i % PD) * SLOT + t * 2048 + 1024);
            } else {
                f.a0[t] = apus_gld<apus_v4u>(ap[t] + q * 128);
                f.a1[t] = apus_gld<apus_v4u>(ap[t] + q * 128 + 64);
            }
            f.s[t] = apus_gld<float>(sp[t] + q);
        }
        /* the waits below count NL loads per group: keep the compiler from
         * merging one group's scale loads with the next group's (adjacent
         * floats of a row) */
        if constexpr (AL) asm volatile("" ::: "memory");
    };
    Grp ring[PD];
#pragma unroll
    for (int i = 0; i < PD; ++i) load(ring[i], i);
    apus_v4f acc[TM];
#pragma unroll
    for (int t = 0; t < TM; ++t) acc[t] = apus_v4f{0.f, 0.f, 0.f, 0.f};
    const int sw = apus_row_swz(r);
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        Grp &cur = ring[i % PD];
        if constexpr (AL) {
            /* group i's loads are complete once only the later groups' are
             * in flight (loads complete in order) */
            const int later = NG - 1 - i < PD - 1 ? NG - 1 - i : PD - 1;
            if (later >= 3) apus_wait_vm<3 * NL>();
            else if (later == 2) apus_wait_vm<2 * NL>();
            else if (later == 1) apus_wait_vm<NL>();
            else apus_wait_vm<0>();
        }
        const apus_v8i b = apus_v8i{(int)cur.b0.x, (int)cur.b0.y, (int)cur.b0.z, (int)cur.b0.w,
                                    (int)cur.b1.x, (int)cur.b1.y, (int)cur.b1.z, (int)cur.b1.w};
        const int sbq = (int)((sbw[i >> 2] >> (8 * (i & 3))) & 0xffu);
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            apus_v4u lo, hi;
            if constexpr (AL) {
                const uint8_t *pp = wring + (i % PD) * SLOT + t * 2048 + r * 128;
                lo = *reinterpret_cast<const apus_v4u *>(pp + ((g ^ sw) << 4));
                hi = *reinterpret_cast<const apus_v4u *>(pp + (((4 + g) ^ sw) << 4));
            } else {
                lo = cur.a0[AL ? 0 : t];
                hi = cur.a1[AL ? 0 : t];
            }
            const apus_v8i a = apus_v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
            acc[t] = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E4M3, 0, 0>(a, b, acc[t], (int)apus_e8m0_of(cur.s[t]),
                                                                         sbq);
        }
        if constexpr (AL) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   /* slot read before refill */
        if (i + PD < NG) load(cur, i + PD);
    }
#pragma unroll
    for (int t = 0; t < TM; ++t) red[wave][t][lane] = acc[t];
    __syncthreads();
    if (wave == 0) {
        /* lane holds D[4g + j][r]: token 16 t + 4 g + j, weight row 16 tile + r;
         * the four K quarters added in order */
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            apus_v4f v = red[0][t][lane];
#pragma unroll
            for (int w = 1; w < 4; ++w) v += red[w][t][lane];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int mm = 16 * t + 4 * g + j;
                if (mm < M) {
                    float x = v[j];
                    if (args.round_out) x = apus_bf16_rne(x);
                    apus_gst<float>(ent.out + (size_t)(ent.o0 + mm) * args.ldo + tile * 16 + r, x);
                }
            }
        }
    }
}

#ifndef APUS_NARROW_PD
#define APUS_NARROW_PD 4
#endif
#ifndef APUS_NARROW_AL
#define APUS_NARROW_AL 1
#endif
template <int NQ, int TM>
bool apus_launch_narrow_tm(const ApusGemmArgs &a, hipStream_t st) {
    constexpr int PD0 = APUS_NARROW_PD, NG = NQ / 4, PD = NG < PD0 ? NG : PD0;
    constexpr bool AL = APUS_NARROW_AL != 0;
    constexpr size_t lds = AL ? (size_t)4 * PD * TM * 2048 : 0;
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void *>(&apus_gemm_narrow_kernel<NQ, TM, PD0, AL>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (attr != hipSuccess) return false;
    hipLaunchKernelGGL((apus_gemm_narrow_kernel<NQ, TM, PD0, AL>), dim3(a.O / 16), dim3(256), lds, st, a);
    return true;
}
template <int NQ>
bool apus_launch_narrow(const ApusGemmArgs &a, hipStream_t st) {
    if (a.ent0.M <= 16) return apus_launch_narrow_tm<NQ, 1>(a, st);
    if (a.ent0.M <= 32) return apus_launch_narrow_tm<NQ, 2>(a, st);
    return apus_launch_narrow_tm<NQ, 4>(a, st);
}

/*
 * Split-K GEMV for dense FP8 and MXFP4 launches with at most 8 rows on
 * tiled weights (the attention's wq_a [1024, 4096] and wkv [512, 4096] at
 * decode, the 4096-row projections at M = 1, one expert's MXFP4 linear:
 * [2048, 4096] fp32 rows 4.1 against 5.0 us per kernel on the few-row
 * schedule). The few-row schedule gives each 16-row
 * tile 4 waves that stream it through a 2-group register ring, so a
 * 512-row weight ran as long as a 1024-row one (4.7 us each): each wave's
 * 16 KB took that long. Here one workgroup of NW waves owns a tile, the
 * waves split K into runs of NG = NQ / NW 128-groups (NG <= 4), and every
 * load of a wave is issued before its first MFMA (a scheduling barrier keeps
 * the compiler from sinking the weight loads below the quantisation).
 * Activations come as codes + scales (ASRC = codes) or as fp32 rows
 * quantised in the wave (ASRC = f32): each (row, group) of the wave's share
 * spread over the 64 lanes, two elements a lane, the group's absolute
 * maximum a wave-wide max, every element rounded to BF16, scaled and
 * converted as in the staging (so the codes are the act-quant kernel's bit
 * for bit), codes and scale byte handed to the fragment lanes through a
 * wave-private LDS slot. Quantising in the fragment layout instead (32
 * elements a lane, one live row in 16) cost ~8 us of SIMD time at
 * [4096, 8192]. Only lanes of rows below M read activation fragments (rows
 * past M are zero and not stored): lanes loading the same address still cost
 * the address unit a lane each. (Codes fetched with one load per 8 / NG rows
 * into the LDS slot instead, as the grouped GEMV does: FP8 [4096, 4096] at
 * M = 1 5.05-5.08 against 5.02-5.04 us, so the fragment loads stay.)
 * Sums: each wave one chain over its groups, the waves added in order in
 * LDS. Splitting a tile over 2-8 workgroups (partial sums through
 * device-coherent stores and a ticket, the last workgroup adding them in
 * order) measured slower at every size: wq_a 5.0-5.4 against 3.8 us, wkv
 * 4.8-5.6 against 3.7.
 */
template <int WF, int NQ, int NW, int ASRC>
__global__ __launch_bounds__(NW * 64) void apus_gemv_split_kernel(ApusGemmArgs args) {
    constexpr int K = NQ * 128, NG = NQ / NW;
    static_assert(NG >= 1 && NQ % NW == 0 && (WF == APUS_W_FP8 || 4 % NG == 0 || NG % 4 == 0), "split shape");
    __shared__ apus_v4f red[NW][64];
    /* fp32 rows: the wave's codes [group][row][128] and scale bytes */
    __shared__ __align__(16) uint8_t lq[ASRC == APUS_A_F32 ? NW : 1][NG][8][128];
    __shared__ uint8_t lsc[ASRC == APUS_A_F32 ? NW : 1][NG][8];
    const ApusGemmEnt ent = args.ent0;
    const int M = ent.M;
    const int tile = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int q0 = wave * NG;
    const bool live = r < M;
    /* the wave's weight stream: FP8 groups of 2 KB (two 16-byte pieces a
     * lane) with 128 x 128 tile scales; MXFP4 groups of 1 KB with the 16
     * scale bytes of the lane's row per 512-slice */
    const ApusWLane wl = apus_wlane<WF>(ent, true, tile * 16 + r, lane, K);
    /* issue order: activations (L2 hits), then the weight stream, then the
     * weight scales; nothing waits before the last load is out (the scale
     * bytes stay per-lane operands: a readfirstlane would wait for them) */
    apus_v4u lo[NG], hi[NG];
    float sa[NG];
    float2 xr[ASRC == APUS_A_F32 ? NG : 1][8];
    if constexpr (ASRC == APUS_A_CODES) {
#pragma unroll
        for (int i = 0; i < NG; ++i) {
            lo[i] = hi[i] = apus_v4u{0u, 0u, 0u, 0u};
            sa[i] = 1.0f;
        }
        if (live) {
            const uint8_t *ap = args.acodes + (size_t)(ent.a0 + r) * K + (size_t)q0 * 128 + g * 16;
            const float *sap = args.ascale + (size_t)(ent.a0 + r) * NQ + q0;
#pragma unroll
            for (int i = 0; i < NG; ++i) {
                lo[i] = apus_gld<apus_v4u>(ap + i * 128);
                hi[i] = apus_gld<apus_v4u>(ap + i * 128 + 64);
                sa[i] = apus_gld<float>(sap + i);
            }
        }
    } else {
        /* fp32 rows: lane l holds elements 2 l, 2 l + 1 of each (row, group) */
        const float *xp = args.ax + (size_t)ent.a0 * K + (size_t)q0 * 128 + 2 * lane;
#pragma unroll
        for (int m = 0; m < 8; ++m)
            if (m < M) {
#pragma unroll
                for (int i = 0; i < NG; ++i) xr[i][m] = apus_gld<float2>(xp + (size_t)m * K + i * 128);
            }
    }
    apus_v4u b0[NG], b1[WF == APUS_W_FP8 ? NG : 1];
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        b0[i] = apus_ld16_stream(wl.w + (size_t)(q0 + i) * wl.qs);
        if constexpr (WF == APUS_W_FP8) b1[i] = apus_ld16_stream(wl.w + (size_t)(q0 + i) * wl.qs + 1024);
    }
    int sb[NG];
    if constexpr (WF == APUS_W_FP8) {
#pragma unroll
        for (int i = 0; i < NG; ++i) sb[i] = (int)apus_gld<uint8_t>(wl.s + q0 + i);
    } else {
        constexpr int NSL = NG < 4 ? 1 : NG / 4;              /* 512-slices of the wave */
        apus_v4u sc4[NSL];
#pragma unroll
        for (int j = 0; j < NSL; ++j) sc4[j] = apus_gld<apus_v4u>(wl.s + (size_t)((q0 >> 2) + j) * wl.ss);
#pragma unroll
        for (int i = 0; i < NG; ++i) {
            const int q = q0 + i;
            sb[i] = (int)((sc4[(q >> 2) - (q0 >> 2)][q & 3] >> (8 * g)) & 0xffu);
        }
    }
    /* keep the scheduler from sinking the weight loads below the
     * quantisation (it would wait for the activations first) */
    __builtin_amdgcn_sched_barrier(0);
    apus_v4f acc = apus_v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        apus_v8i a;
        int ea;
        if constexpr (ASRC == APUS_A_CODES) {
            a = apus_v8i{(int)lo[i].x, (int)lo[i].y, (int)lo[i].z, (int)lo[i].w,
                         (int)hi[i].x, (int)hi[i].y, (int)hi[i].z, (int)hi[i].w};
            ea = (int)apus_e8m0_of(sa[i]);
        } else {
            /* quantise the group's M rows across the wave (two elements a
             * lane), codes and scale bytes through the wave's LDS slot, then
             * the fragment of lane (r, g) from row r */
#pragma unroll
            for (int m = 0; m < 8; ++m)
                if (m < M) {
                    const float v0 = apus_bf16_rne(xr[i][m].x), v1 = apus_bf16_rne(xr[i][m].y);
                    /* seeded with 0 as the staging's max: a group of NaN only
                     * gets 0, not NaN */
                    const float amax = apus_wave_max_dpp(fmaxf(fmaxf(0.0f, fabsf(v0)), fabsf(v1)));
                    const uint32_t e = apus_act_scale_exp(amax);
                    const float inv = apus_inv_pow2_from_exp(e);
                    reinterpret_cast<uint16_t *>(lq[wave][i][m])[lane] =
                        (uint16_t)apus_e4m3_pack2_hw(v0 * inv, v1 * inv);
                    if (lane == 0) lsc[wave][i][m] = (uint8_t)e;
                }
            apus_v4u l4 = apus_v4u{0u, 0u, 0u, 0u}, h4 = l4;
            ea = 127;
            if (live) {
                l4 = *reinterpret_cast<const apus_v4u *>(&lq[wave][i][r][16 * g]);
                h4 = *reinterpret_cast<const apus_v4u *>(&lq[wave][i][r][64 + 16 * g]);
                ea = lsc[wave][i][r];
            }
            a = apus_v8i{(int)l4.x, (int)l4.y, (int)l4.z, (int)l4.w, (int)h4.x, (int)h4.y, (int)h4.z, (int)h4.w};
        }
        if constexpr (WF == APUS_W_FP8) {
            const apus_v8i b = apus_v8i{(int)b0[i].x, (int)b0[i].y, (int)b0[i].z, (int)b0[i].w,
                                        (int)b1[i].x, (int)b1[i].y, (int)b1[i].z, (int)b1[i].w};
            acc = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E4M3, 0, 0>(a, b, acc, ea, sb[i]);
        } else {
            const apus_v8i b = apus_v8i{(int)b0[i].x, (int)b0[i].y, (int)b0[i].z, (int)b0[i].w, 0, 0, 0, 0};
            acc = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E2M1, 0, 0>(a, b, acc, ea, sb[i]);
        }
    }
    if constexpr (NW > 1) {
        red[wave][lane] = acc;
        __syncthreads();
        if (wave != 0) return;
        acc = red[0][lane];
#pragma unroll
        for (int w = 1; w < NW; ++w) acc += red[w][lane];
    }
    /* lane holds D[4 g + j][r]: row 4 g + j, weight row 16 tile + r */
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int mm = 4 * g + j;
        if (mm < M) {
            float x = acc[j];
            if (args.round_out) x = apus_bf16_rne(x);
            apus_gst<float>(ent.out + (size_t)(ent.o0 + mm) * args.ldo + tile * 16 + r, x);
        }
    }
}

/* waves per workgroup of the split-K GEMV: one 128-group a wave where 16
 * waves cover K (K <= 2048), else NQ / 16. Measured (us, wq_a / wkv /
 * wo_b / wq_b fp32-row linears, FP8 [4096, 4096] codes at M = 1): 1 group
 * 3.85 / 3.75 / 8.4 / 7.5 / 4.85; at most 2 (fp32) / 4 (codes) 3.85 / 3.77 /
 * 8.5 / 7.75 / 5.2; 4 groups for fp32 4.2 / 4.1 / 8.5 / 8.0 */
#ifndef APUS_SPLIT_FP4
#define APUS_SPLIT_FP4 1
#endif
#ifndef APUS_SPLIT_NG_CODES
#define APUS_SPLIT_NG_CODES 1
#endif
#ifndef APUS_SPLIT_NG_F32
#define APUS_SPLIT_NG_F32 1
#endif
template <int WF, int NQ, int ASRC>
void apus_launch_split_k(const ApusGemmArgs &a, hipStream_t st) {
    constexpr int NW0 = NQ / (ASRC == APUS_A_F32 ? APUS_SPLIT_NG_F32 : APUS_SPLIT_NG_CODES);
    constexpr int NW = NW0 < 1 ? 1 : NW0 > 16 ? 16 : NW0;
    static_assert(NQ / NW <= 4, "at most 4 groups a wave");
    hipLaunchKernelGGL((apus_gemv_split_kernel<WF, NQ, NW, ASRC>), dim3(a.O / 16), dim3(NW * 64), 0, st, a);
}
template <int WF, int ASRC>
void apus_launch_split(const ApusGemmArgs &a, hipStream_t st) {
    switch (a.K) {
    case 1024: apus_launch_split_k<WF, 8, ASRC>(a, st); break;
    case 2048: apus_launch_split_k<WF, 16, ASRC>(a, st); break;
    case 4096: apus_launch_split_k<WF, 32, ASRC>(a, st); break;
    default:   apus_launch_split_k<WF, 64, ASRC>(a, st); break;
    }
}

/*
 * Grouped GEMV for grouped launches of tiled MXFP4 / FP8 entries with at most
 * 8 rows each and no required accumulation order (config 0: twelve
 * [2048, 4096] MXFP4 GEMVs at M = 1). One workgroup of NW waves owns a
 * (16-row weight tile, entry); each wave takes a contiguous run of NG
 * 128-groups (8 KB of weight bytes) and issues all its loads before its
 * first MFMA; the waves' sums are added in order in LDS.
 * Activations: each wave fetches its groups of each live row with one
 * contiguous load instruction per row (64 lanes x 16 bytes) into a
 * wave-private LDS slot and reads its fragments from there. Measured on the
 * config-0 launch shape (standalone, 53.6 MB per launch, fresh copies): the
 * weight stream alone with this shape 9.1 us; fragments loaded straight from
 * the codes by the lanes of live rows (a dozen 4-lane loads per wave) 11.7
 * us; through one load per row and LDS 9.9 us (the cost is per load
 * instruction, not per byte). In the library the launch takes 10.6-10.8 us
 * against 11.3-11.7 on the few-row schedule, which runs one whole-K wave per
 * tile through a register ring and stages 8 activation rows per workgroup
 * whatever M is; 4 KB waves (8 per tile) and 4-lane fragment loads measured
 * 11.9 us.
 */
template <int WF, int NQ, int NW, int MR>
__global__ __launch_bounds__(NW * 64) void apus_gemv_grp_kernel(ApusGemmArgs args) {
    constexpr int K = NQ * 128, NG = NQ / NW;
    static_assert(NQ % NW == 0 && NG * 16 <= 128 && NG % 4 == 0, "grouped GEMV shape");
    __shared__ apus_v4f red[NW][64];
    /* MR: rows an entry may have (1 or 8) */
    __shared__ __align__(16) uint8_t lx[NW][MR][NG * 128];     /* wave's codes [row][group bytes] */
    __shared__ float lsa[NW][MR][NG];
    /* grouped launches only: the entry straight from the table (the generic
     * lookup's checks cost dependent scalar loads before the first address) */
    const ApusGemmEnt ent = args.ents[blockIdx.y];
    /* every field in one batch of scalar loads: else the early return below
     * costs a round trip of its own for M (config-0 launch 10.7-10.8 against
     * 10.9 us; pinning the kernel arguments the same way turned the entry
     * fetch into vector loads, 11.3-11.4 us) */
    asm volatile("" ::"s"(ent.w), "s"(ent.ws), "s"(ent.out), "s"(ent.arows), "s"(ent.orows), "s"(ent.a0),
                 "s"(ent.o0), "s"(ent.M));
    /* entries past the launch's row bound are skipped, as on the few-row
     * schedule */
    const int M = ent.M;
    if (M <= 0 || M > MR) return;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int tile = blockIdx.x, o = tile * 16 + r;
    const int q0 = wave * NG;
    /* activation rows first (L2 hits: they return before the weights, and
     * their LDS hand-off runs while the weights stream): row m's NG groups
     * are NG * 128 contiguous bytes, one load instruction; the M x NG scales
     * one more. Row indices of a gathered entry: one load, lane m. */
    constexpr int XL = NG * 8;                                  /* lanes of one row's load */
    apus_v4u xv[MR];
    float xsv = 0.0f;
    if (ent.arows) {
        /* gathered rows: the indices first (one round trip) */
        const int rv = lane < M ? apus_gld<int>(ent.arows + lane) : 0;
        const int srow = __shfl(rv, lane / NG, 64);
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            if (m < M && lane < XL) {
                const int row = __builtin_amdgcn_readlane(rv, m);
                xv[m] = apus_gld<apus_v4u>(args.acodes + (size_t)row * K + (size_t)q0 * 128 + lane * 16);
            }
        }
        if (lane < M * NG) xsv = apus_gld<float>(args.ascale + (size_t)srow * NQ + q0 + lane % NG);
    } else {
        const uint8_t *xa = args.acodes + (size_t)ent.a0 * K + (size_t)q0 * 128 + lane * 16;
#pragma unroll
        for (int m = 0; m < MR; ++m)
            if (m < M && lane < XL) xv[m] = apus_gld<apus_v4u>(xa + (size_t)m * K);
        if (lane < M * NG) xsv = apus_gld<float>(args.ascale + (size_t)(ent.a0 + lane / NG) * NQ + q0 + lane % NG);
    }
    const ApusWLane wl = apus_wlane<WF>(ent, true, o, lane, K);
    apus_v4u b0[NG], b1[WF == APUS_W_FP8 ? NG : 1];
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        b0[i] = apus_ld16_stream(wl.w + (size_t)(q0 + i) * wl.qs);
        if constexpr (WF == APUS_W_FP8) b1[i] = apus_ld16_stream(wl.w + (size_t)(q0 + i) * wl.qs + 1024);
    }
    apus_v4u sc4[WF == APUS_W_FP4 ? NG / 4 : 1];
    unsigned sc1[WF == APUS_W_FP8 ? NG : 1];
    if constexpr (WF == APUS_W_FP4) {
        /* the 16 scale bytes of the lane's row per 512-slice */
#pragma unroll
        for (int j = 0; j < NG / 4; ++j) sc4[j] = apus_gld<apus_v4u>(wl.s + (size_t)((q0 >> 2) + j) * wl.ss);
    } else {
#pragma unroll
        for (int i = 0; i < NG; ++i) sc1[i] = apus_gld<uint8_t>(wl.s + q0 + i);
    }
    /* activation rows to the wave's LDS slot, then every lane's fragments */
#pragma unroll
    for (int m = 0; m < MR; ++m)
        if (m < M && lane < XL) *reinterpret_cast<apus_v4u *>(&lx[wave][m][lane * 16]) = xv[m];
    if (lane < M * NG) (&lsa[wave][0][0])[lane] = xsv;
    const bool live = r < M;
    const int rr = live ? r : 0;
    apus_v8i av[NG];
    int ea[NG];
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        const apus_v4u l4 = *reinterpret_cast<const apus_v4u *>(&lx[wave][rr][i * 128 + g * 16]);
        const apus_v4u h4 = *reinterpret_cast<const apus_v4u *>(&lx[wave][rr][i * 128 + 64 + g * 16]);
        const int z = live ? -1 : 0;
        av[i] = apus_v8i{(int)l4.x & z, (int)l4.y & z, (int)l4.z & z, (int)l4.w & z,
                         (int)h4.x & z, (int)h4.y & z, (int)h4.z & z, (int)h4.w & z};
        ea[i] = live ? (int)apus_e8m0_of(lsa[wave][rr][i]) : 127;
    }
    apus_v4f acc = apus_v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        if constexpr (WF == APUS_W_FP4) {
            const int sb = (int)((sc4[i >> 2][i & 3] >> (8 * g)) & 0xffu);
            const apus_v8i b = apus_v8i{(int)b0[i].x, (int)b0[i].y, (int)b0[i].z, (int)b0[i].w, 0, 0, 0, 0};
            acc = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E2M1, 0, 0>(av[i], b, acc, ea[i], sb);
        } else {
            const apus_v8i b = apus_v8i{(int)b0[i].x, (int)b0[i].y, (int)b0[i].z, (int)b0[i].w,
                                        (int)b1[i].x, (int)b1[i].y, (int)b1[i].z, (int)b1[i].w};
            acc = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E4M3, 0, 0>(av[i], b, acc, ea[i], (int)sc1[i]);
        }
    }
    if constexpr (NW > 1) {
        red[wave][lane] = acc;
        __syncthreads();
        if (wave != 0) return;
        acc = red[0][lane];
#pragma unroll
        for (int w = 1; w < NW; ++w) acc += red[w][lane];
    }
    /* lane holds D[4 g + j][r]: row 4 g + j, weight row o */
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int mm = 4 * g + j;
        if (mm < M) {
            float x = acc[j];
            if (args.round_out) x = apus_bf16_rne(x);
            const int orow = ent.orows ? apus_gld<int>(ent.orows + mm) : ent.o0 + mm;
            apus_gst<float>(ent.out + (size_t)orow * args.ldo + o, x);
        }
    }
}

/* 8 KB of weight bytes a wave: FP4 8 groups (4 waves at K = 4096, 2 at
 * 2048), FP8 4 groups. Not used for the routed dispatch: its few-row tables
 * have a slot per expert (up to 256, mostly empty at config 2), and a
 * workgroup per (tile, slot) that reads its entry before it can leave made
 * the K-quarter w2 (whose order 4 waves of a quarter each would keep bit
 * for bit) twice as slow: config 2 874 against 440 us. */
template <int WF, int NQ>
void apus_launch_grp_k(const ApusGemmArgs &a, int n_ent, hipStream_t st) {
    constexpr int NG = WF == APUS_W_FP4 ? 8 : 4;
    constexpr int NW = NQ / NG;
    if (a.max_m == 1)
        hipLaunchKernelGGL((apus_gemv_grp_kernel<WF, NQ, NW, 1>), dim3(a.O / 16, n_ent), dim3(NW * 64), 0, st, a);
    else
        hipLaunchKernelGGL((apus_gemv_grp_kernel<WF, NQ, NW, 8>), dim3(a.O / 16, n_ent), dim3(NW * 64), 0, st, a);
}
template <int WF>
void apus_launch_grp(const ApusGemmArgs &a, int n_ent, hipStream_t st) {
    if (a.K == 4096) apus_launch_grp_k<WF, 32>(a, n_ent, st);
    else             apus_launch_grp_k<WF, 16>(a, n_ent, st);
}

/* launch the LDS tile schedule (returns false where it does not apply) */
template <int NQ>
bool apus_launch_lds_tile(const ApusGemmArgs &a, hipStream_t st) {
    constexpr int NST = APUS_LT_NST < NQ ? APUS_LT_NST : NQ;
    constexpr size_t lds = (size_t)NST * (64 + 128) * 128 + 64 * NQ * 4;
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void *>(&apus_gemm_lds_kernel<NQ>), hipFuncAttributeMaxDynamicSharedMemorySize,
        (int)lds);
    if (attr != hipSuccess) return false;
    const int tiles = (a.ent0.M + 63) / 64 * (a.O / 128);
    hipLaunchKernelGGL(apus_gemm_lds_kernel<NQ>, dim3(tiles), dim3(512), lds, st, a);
    return true;
}

/*
 * LDS many-row schedule for the routed MXFP4 experts (grouped launches from
 * the route kernel's work list, MFMA-tiled weights, K 2048 / 4096): one
 * workgroup per (64-row chunk of an expert, 128 weight rows), whole K, both
 * operands global -> LDS through NST stages of one 128-group as in
 * apus_gemm_lds_kernel: per stage 8 loads of 8 gathered activation rows
 * (row table of the entry) and 8 loads of 1 KB weight fragments (FP4: a
 * 16-row tile's 128-group is 1 KB); the weight scales of the 8 tiles (one
 * contiguous block) and the chunk's activation scales go to LDS up front.
 * 8 waves of 16 chunk rows x 64 weight rows; waves whose 16 rows lie past
 * the chunk's end skip their MFMAs. Accumulation per output: one chain over
 * the 128-groups (w1/w3), or with FOLD four chains from zero over the
 * quarters of K added left to right (w2), the orders of the one-token
 * kernels, so results equal the other schedules bit for bit.
 */
template <int NS, bool FOLD, int NST>
__global__ __launch_bounds__(512, 2) void apus_gemm_prefill_lds_kernel(ApusGemmArgs args) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int K = NS * 512, NQ = NS * 4, ROWS = 64;
    constexpr int AB = ROWS * 128, STB = AB + 8 * 1024;
    constexpr int SCB = 8 * NS * 256;                          /* weight scales of 8 tiles */
    static_assert(!FOLD || NS == 4, "K-quarter order at K = 2048");
    static_assert(NQ % 8 == 0 && SCB % 8192 == 0, "loads per wave");
    const int2 it = apus_gld<int2>(args.items + blockIdx.y);
    if (it.x < 0) return;
    const ApusGemmEnt ent = apus_gld<ApusGemmEnt>(args.ents + it.x);
    if (ent.M <= args.m_min || (args.m_max > 0 && ent.M > args.m_max)) return;
    const int c0 = it.y;
    const int rows = min(ROWS, ent.M - c0);
    const int n0 = blockIdx.x * 128;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int wm = wave >> 1, wn = wave & 1;
    uint8_t *lws = lds + NST * STB;                            /* [8 tiles][NS][16 rows][16 B] */
    float *lsa = reinterpret_cast<float *>(lws + SCB);         /* [q][64 rows] fp32 */
    const unsigned lbase = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds);
    auto arow_of = [&](int lr) {
        const int mm = c0 + (lr < rows ? lr : rows - 1);
        return ent.arows ? apus_gld<int>(ent.arows + mm) : ent.a0 + mm;
    };
    /* stage loads of this wave: activation instruction `wave` (8 rows:
     * lane -> row 8 wave + lane / 8, LDS slot lane % 8 holding 16-byte chunk
     * (lane % 8) ^ swizzle(row)) and weight tile `wave` */
    const int alr = 8 * wave + (lane >> 3);
    const int asw = apus_row_swz(alr);
    const uint8_t *asrc = args.acodes + (size_t)arow_of(alr) * K + ((lane & 7) ^ asw) * 16;
    const uint8_t *bsrc = ent.w + ((size_t)((n0 >> 4) + wave) * NQ) * 1024 + lane * 16;
    auto issue = [&](int q, int slot) {
        apus_g2lds16(asrc + q * 128, lbase + slot * STB + wave * 1024);
        apus_g2lds16(bsrc + q * 1024, lbase + slot * STB + AB + wave * 1024);
    };
    /* up front: the weight scales (8 tiles x NS slices x 256 B, contiguous)
     * and the activation scales of the chunk (one dword load per group and
     * 64 rows) */
    const uint8_t *wsrc = ent.ws + (size_t)(n0 >> 4) * NS * 256;
#pragma unroll
    for (int u = 0; u < SCB / 8192; ++u)
        apus_g2lds16(wsrc + (size_t)(u * 8 + wave) * 1024 + lane * 16, lbase + NST * STB + (u * 8 + wave) * 1024);
    const int srow = arow_of(lane);
#pragma unroll
    for (int u = 0; u < NQ / 8; ++u) {
        const int q = u * 8 + wave;
        apus_g2lds4(args.ascale + (size_t)srow * NQ + q, lbase + NST * STB + SCB + q * ROWS * 4);
    }
#pragma unroll
    for (int st = 0; st < NST; ++st) issue(st, st);
    constexpr int PRE = SCB / 8192 + NQ / 8;                   /* up-front loads of a wave */
    (void)PRE;

    apus_v4f acc[4], tot[FOLD ? 4 : 1];
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = apus_v4f{0.f, 0.f, 0.f, 0.f};
    if constexpr (FOLD) {
#pragma unroll
        for (int i = 0; i < 4; ++i) tot[i] = apus_v4f{-0.f, -0.f, -0.f, -0.f};
    }
    const bool live = wm * 16 < rows;                          /* wave-uniform */
    const int arow = wm * 16 + r;
    const int sw = apus_row_swz(r);
    struct Frag { apus_v8i a; apus_v4u b[4]; int sa; unsigned sb[4]; };
    auto read_frag = [&](Frag &f, int q) {
        const uint8_t *stg = lds + (q % NST) * STB;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int tl = wn * 4 + i;
            f.b[i] = *reinterpret_cast<const apus_v4u *>(stg + AB + tl * 1024 + lane * 16);
            f.sb[i] = *reinterpret_cast<const unsigned *>(lws + (tl * NS + (q >> 2)) * 256 + r * 16 + (q & 3) * 4);
        }
        const uint8_t *p = stg + arow * 128;
        const apus_v4u lo = *reinterpret_cast<const apus_v4u *>(p + ((g ^ sw) << 4));
        const apus_v4u hi = *reinterpret_cast<const apus_v4u *>(p + (((4 + g) ^ sw) << 4));
        f.a = apus_v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        f.sa = (int)apus_e8m0_of(lsa[q * ROWS + arow]);
    };
    /* stage q is in LDS once at most (stages issued after it) x 2 loads are
     * in flight: NST - 1 stages follow stage 0 before the loop (which also
     * covers the up-front scale loads, issued first); in the loop
     * stage_ready(q) runs before stage q + NST - 1 is issued */
    auto stage_ready = [&](int q) {
        const int last = q == 0 ? NST - 1 : (q + NST - 2 < NQ - 1 ? q + NST - 2 : NQ - 1);
        const int ahead = last - q;
        if (ahead >= 3) apus_wait_vm<6>();
        else if (ahead == 2) apus_wait_vm<4>();
        else if (ahead == 1) apus_wait_vm<2>();
        else apus_wait_vm<0>();
        apus_lds_barrier();
    };
    static_assert(NST <= 4 && NST <= NQ, "stage_ready waits for at most 3 stages ahead");
    Frag fr[2];
    stage_ready(0);
    read_frag(fr[0], 0);
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        if (q + 1 < NQ) {
            stage_ready(q + 1);
            if (q + NST < NQ) issue(q + NST, (q + NST) % NST);
            read_frag(fr[(q + 1) & 1], q + 1);
        }
        const Frag &f = fr[q & 1];
        if (live) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const apus_v8i b = apus_v8i{(int)f.b[i].x, (int)f.b[i].y, (int)f.b[i].z, (int)f.b[i].w, 0, 0, 0, 0};
                acc[i] = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E2M1, 0, 0>(f.a, b, acc[i], f.sa,
                                                                             (int)((f.sb[i] >> (8 * g)) & 0xffu));
            }
        }
        if constexpr (FOLD) {
            if ((q & 3) == 3) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    tot[i] += acc[i];
                    acc[i] = apus_v4f{0.f, 0.f, 0.f, 0.f};
                }
            }
        }
    }
    if (!live) return;
    /* lane holds D[4g + j][r]: chunk row 16 wm + 4 g + j, weight row n0 + 64 wn + 16 i + r */
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int lr = wm * 16 + 4 * g + j;
        if (lr < rows) {
            const int mm = c0 + lr;
            const int orow = ent.orows ? apus_gld<int>(ent.orows + mm) : ent.o0 + mm;
            float *d = ent.out + (size_t)orow * args.ldo + n0 + wn * 64 + r;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float v = FOLD ? tot[FOLD ? i : 0][j] : acc[i][j];
                if (args.round_out) v = apus_bf16_rne(v);
                apus_gst<float>(d + i * 16, v);
            }
        }
    }
}

/* launch the LDS many-row schedule over a work list (returns false where it
 * does not apply) */
template <int NS, bool FOLD>
bool apus_launch_pre_lds(const ApusGemmArgs &p, int n_items, hipStream_t st) {
    constexpr int NST = APUS_PRE_LDS_NST;
    constexpr size_t lds = (size_t)NST * (64 * 128 + 8 * 1024) + 8 * NS * 256 + 64 * NS * 4 * 4;
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void *>(&apus_gemm_prefill_lds_kernel<NS, FOLD, NST>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (attr != hipSuccess || p.O % 128 || !p.wtiled) return false;
    hipLaunchKernelGGL((apus_gemm_prefill_lds_kernel<NS, FOLD, NST>), dim3(p.O / 128, n_items), dim3(512), lds,
                       st, p);
    return true;
}

/*
 * One-token MoE dispatch kernels (few routed pairs, MXFP4 experts; with SH,
 * also the FP8 shared expert of each token in the same two launches).
 *
 * w1/w3 (apus_moe_pair13_kernel): a workgroup owns 32 rows of inter for one
 * pair; each wave streams one 16-row tile of w1 or w3 over the whole K (one
 * accumulation chain, as the few-row schedule without a K split); the pair's
 * x row is quantised once while staging. The epilogue meets g and u in LDS
 * and writes h = swiglu(bf16 g, bf16 u) (c/moe.h:113-126, :198-209). With SH,
 * launch rows npairs + t do the same for token t's shared expert (FP8 w1/w3,
 * c/moe.h:570-585) and write its h to h row npairs + t.
 *
 * w2 (apus_moe_pair2_kernel): a workgroup owns 16 columns of dim and, token by
 * token, multiplies the token's NP = topk staged h rows against their experts'
 * weights; the 4 waves split K in quarters and their partial sums meet in LDS
 * (added in part order), then y[t, o] = sum_j wgt * bf16(eo_j) in j order
 * (c/moe.h:148-158, :447-449). The weight ring runs across the pairs, so the
 * whole tile's weights are in flight at once; nothing leaves the workgroup but
 * y. With SH, the token's shared h is staged as row NP and multiplied by the
 * FP8 shared w2 in the same workgroup: sh = bf16(w2 h) and the sublayer
 * output bf16(y + sh) (c/moe.h:588-589) are written too.
 */
template <int WF, int NS, int TILES>
__device__ __forceinline__ void apus_pair13_body(const ApusGemmArgs &args, const ApusStageRaw<APUS_A_F32> &raw,
                                                 const ApusGemmEnt &ent, bool tiled, bool ok,
                                                 int hrow, uint8_t *lcodes, uint8_t *lsc,
                                                 float (*lgu)[TILES][64], float *plain = nullptr) {
    constexpr int K = NS * 512;
    /* 16-wave workgroups get at most 128 registers a lane: a shorter FP8 ring */
    constexpr int PD = (TILES == 8 && WF == APUS_W_FP8) ? 2 : 3;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int mat = wave & 1, tile = wave >> 1;
    const int o = blockIdx.x * (16 * TILES) + tile * 16 + r;
    const ApusWLane wl = apus_wlane<WF>(ent, tiled, o, lane, K);
    ApusBFrag<WF> ring[PD];
#pragma unroll
    for (int u = 0; u < PD; ++u) apus_load_b_full<WF>(ring[u], wl, u);
    apus_stage_quant<K, APUS_A_F32>(args, raw, lcodes, lsc);
    apus_lds_barrier();
    /* A row 0 is the pair's x; the other 15 rows are zero */
    const int z = r == 0 ? -1 : 0;
    const uint8_t *arow = lcodes + g * 16;
    apus_v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        ApusBFrag<WF> &cur = ring[s % PD];
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const int q = s * 4 + st;
            const uint4 a0 = *reinterpret_cast<const uint4 *>(arow + q * 128);
            const uint4 a1 = *reinterpret_cast<const uint4 *>(arow + q * 128 + 64);
            const apus_v8i a = apus_v8i{(int)a0.x & z, (int)a0.y & z, (int)a0.z & z, (int)a0.w & z,
                                        (int)a1.x & z, (int)a1.y & z, (int)a1.z & z, (int)a1.w & z};
            if constexpr (WF == APUS_W_FP4) {
                const apus_v4u w = cur.w[st][0];
                const apus_v8i b = apus_v8i{(int)w.x, (int)w.y, (int)w.z, (int)w.w, 0, 0, 0, 0};
                const int sb = (int)((cur.s[st] >> (8 * g)) & 0xffu);
                acc = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E2M1, 0, 0>(a, b, acc, (int)lsc[q], sb);
            } else {
                const apus_v4u w0 = cur.w[st][0], w1 = cur.w[st][1];
                const apus_v8i b = apus_v8i{(int)w0.x, (int)w0.y, (int)w0.z, (int)w0.w,
                                            (int)w1.x, (int)w1.y, (int)w1.z, (int)w1.w};
                acc = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E4M3, 0, 0>(a, b, acc, (int)lsc[q],
                                                                           (int)cur.s[st]);
            }
        }
        if (s + PD < NS) apus_load_b_full<WF>(cur, wl, s + PD);
    }
    /* lane (g 0, r) holds D[0][r]: this pair, inter column o. Every lane
     * stores its element (a lane-dependent store as the only consumer of the
     * MFMA results would pull them into a narrowed EXEC); 32 threads then
     * pick the g == 0 lanes of the w1 and w3 waves */
    lgu[mat][tile][lane] = apus_bf16_rne(acc[0]);
    __syncthreads();
    if (plain) {
        /* a dense linear riding in the launch: rows [0, O) of its weight are
         * "w1", rows [O, 2 O) "w3"; out = bf16(W x) as is */
        if (threadIdx.x < 32 * TILES) {
            const int mt = threadIdx.x / (16 * TILES), rem = threadIdx.x - mt * 16 * TILES;
            const int t = rem >> 4, rr = rem & 15;
            apus_gst<float>(plain + (size_t)mt * args.O + blockIdx.x * (16 * TILES) + t * 16 + rr,
                            lgu[mt][t][rr]);
        }
        return;
    }
    if constexpr (TILES == 8) {
        /* the workgroup holds a whole 128-column group of h: quantise it
         * here as the activation quantiser does (c/fp4.h:293-321: BF16,
         * amax, E8M0 scale, E4M3 codes); threads 0..127 own one column */
        __shared__ float lmax[2];
        const int t = threadIdx.x >> 4, rr = threadIdx.x & 15;
        float h = 0.0f;
        if (threadIdx.x < 128)
            h = ok ? apus_swiglu_h(lgu[0][t & 7][rr], lgu[1][t & 7][rr], args.limit) : 0.0f;
        const float m = apus_wave_max(fabsf(h));
        if (threadIdx.x < 128 && (threadIdx.x & 63) == 0) lmax[threadIdx.x >> 6] = m;
        __syncthreads();
        if (threadIdx.x < 128) {
            const uint32_t e = apus_act_scale_exp(fmaxf(lmax[0], lmax[1]));
            const float inv = apus_inv_pow2_from_exp(e);
            const int G = args.O >> 7;
            apus_gst<uint8_t>(args.hq + (size_t)hrow * args.O + blockIdx.x * 128 + threadIdx.x,
                              (uint8_t)apus_e4m3_pack2_hw(h * inv, 0.0f));
            if (threadIdx.x == 0) apus_gst<uint8_t>(args.hqs + (size_t)hrow * G + blockIdx.x, (uint8_t)e);
        }
        return;
    }
    float *hdst = args.pout[0] + (size_t)hrow * args.O;
    if (threadIdx.x < 32) {
        const int t = threadIdx.x >> 4, rr = threadIdx.x & 15;
        const float h = ok ? apus_swiglu_h(lgu[0][t][rr], lgu[1][t][rr], args.limit) : 0.0f;
        float *dst = hdst + blockIdx.x * 32 + t * 16 + rr;
        if (args.hq) /* device-coherent: the group's last workgroup reads it */
            __hip_atomic_store(dst, h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
            apus_gst<float>(dst, h);
    }
    if (!args.hq) return;
    /* The four workgroups of a 128-column group take tickets once their h
     * stores have completed; the last one quantises the group as the
     * activation quantiser does (c/fp4.h:293-321: BF16, amax, E8M0 scale,
     * E4M3 codes), reading the h values with device-coherent loads, and
     * returns the counter to zero for the next launch. */
    __shared__ int last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    const int G = args.O >> 7, gq = blockIdx.x >> 2;
    unsigned *tk = args.hq_tk + (size_t)hrow * G + gq;
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(tk, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 3u;
    __syncthreads();
    if (!last || threadIdx.x >= 8) return;
    const float *src = hdst + gq * 128 + threadIdx.x * 16;
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i)
        v[i] = apus_bf16_rne(__hip_atomic_load(src + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) m = fmaxf(m, fabsf(v[i]));
    m = fmaxf(m, __shfl_xor(m, 1, 64));
    m = fmaxf(m, __shfl_xor(m, 2, 64));
    m = fmaxf(m, __shfl_xor(m, 4, 64));
    const uint32_t e = apus_act_scale_exp(m);
    const float inv = apus_inv_pow2_from_exp(e);
    uint32_t w4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        w4[i] = apus_e4m3_pack4_hw(v[4 * i] * inv, v[4 * i + 1] * inv, v[4 * i + 2] * inv,
                                   v[4 * i + 3] * inv);
    apus_gst<apus_v4u>(args.hq + (size_t)hrow * args.O + gq * 128 + threadIdx.x * 16,
                       apus_v4u{w4[0], w4[1], w4[2], w4[3]});
    if (threadIdx.x == 0) {
        apus_gst<uint8_t>(args.hqs + (size_t)hrow * G + gq, (uint8_t)e);
        __hip_atomic_store(tk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int NS, bool SH, int TILES>
__global__ __launch_bounds__(128 * TILES) void apus_moe_pair13_kernel(ApusGemmArgs args) {
    constexpr int K = NS * 512, NQ = NS * 4, LDK = K + 32;
    __shared__ __align__(16) uint8_t lcodes[LDK];
    __shared__ uint8_t lsc[NQ];
    __shared__ float lgu[2][TILES][64];        /* [mat][tile][lane] */
    if (args.zero && blockIdx.y == 0) {
        for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < args.nzero; i += gridDim.x * blockDim.x)
            args.zero[i] = 0u;
    }
    const int mat = (threadIdx.x >> 6) & 1;
    const int p = blockIdx.y;
    ApusStageRaw<APUS_A_F32> raw;
    const int nsh = SH ? args.acc_s : 0;
    if (args.rdout && p >= args.npairs + nsh) {
        /* token t's dense FP8 linear [2 O, K] (rider rows after the pairs and
         * the shared-expert rows): out row t of rdout [s, 2 O] */
        const int t = p - args.npairs - nsh;
        apus_stage_load<K, APUS_A_F32>(args, nullptr, t, 0, 1, 0, raw);
        ApusGemmEnt ent;
        ent.w = mat ? args.rdw + (size_t)args.O * K : args.rdw;
        ent.ws = mat ? args.rdws + (size_t)(args.O / 128) * NQ : args.rdws;
        apus_pair13_body<APUS_W_FP8, NS, TILES>(args, raw, ent, args.rdtiled, true, p, lcodes, lsc, lgu,
                                                args.rdout + (size_t)t * 2 * args.O);
        return;
    }
    if (SH && p >= args.npairs) {
        /* token t's shared expert: FP8 w1 / w3 */
        const int t = p - args.npairs;
        apus_stage_load<K, APUS_A_F32>(args, nullptr, t, 0, 1, 0, raw);
        ApusGemmEnt ent;
        ent.w = mat ? args.shw[2] : args.shw[0];
        ent.ws = mat ? args.shws[2] : args.shws[0];
        apus_pair13_body<APUS_W_FP8, NS, TILES>(args, raw, ent, args.sh_tiled, true, p, lcodes, lsc, lgu);
        return;
    }
    /* the pair's x row: its loads go out first */
    apus_stage_load<K, APUS_A_F32>(args, nullptr, p / args.adiv, 0, 1, 0, raw);
    int e;
    if (args.rsp) {
        __shared__ __align__(16) uint64_t lk[1024];
        __shared__ int32_t chosen[16];
        __shared__ float chp[16];
        const int t = p / args.adiv, j = p - t * args.adiv;
        apus_route_token(args.rt2e ? nullptr : args.rsel + (size_t)t * args.rE,
                         args.rsp + (size_t)t * args.rE, args.rE, args.adiv,
                         args.rt2e ? args.rt2e + apus_gld<int64_t>(args.rids + t) * args.adiv : nullptr,
                         lk, chosen, chp);
        e = chosen[j];
        if (blockIdx.x == 0 && threadIdx.x == 0) {
            apus_gst<int>(args.ridx + p, e);
            apus_gst<float>(args.rwgt + p, apus_route_weight(chp, args.adiv, j, args.rscale));
        }
    } else {
        e = apus_gld<int>(args.pidx + p);
    }
    const bool ok = (unsigned)e < (unsigned)args.pE;
    ApusGemmEnt ent;
    apus_expert_ptrs(args, mat, ok ? e : 0, ent.w, ent.ws);
    apus_pair13_body<APUS_W_FP4, NS, TILES>(args, raw, ent, args.wtiled, ok, p, lcodes, lsc, lgu);
}

template <int NS, int NP, bool SH, int G>
__global__ __launch_bounds__(256 * G) void apus_moe_pair2_kernel(ApusGemmArgs args) {
    /* G groups of 4 waves: group i takes the pairs [i NP/G, (i+1) NP/G) (and
     * the last group the shared w2); the 4 waves of a group take the K
     * quarters */
    constexpr int K = NS * 512, NQ = NS * 4, KS = 4, NSW = NS / KS, NPG = NP / G;
    constexpr int STEPS = NPG * NSW, PD = STEPS < 6 ? STEPS : (NSW == 1 ? 6 : 4);
    static_assert(NP % G == 0, "pairs per wave group");
    constexpr int NR = NP + (SH ? 1 : 0);            /* A rows per token */
    static_assert(NS % KS == 0 && NP <= 8, "pair2 shape");
    static_assert(!SH || NSW == 1, "the shared w2 takes one 512-slice per wave");
    __shared__ float lred[KS][NR][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int kpart = wave & 3, grp = __builtin_amdgcn_readfirstlane(wave >> 2), jb = grp * NPG;
    const bool shg = SH && grp == G - 1;           /* this group runs the shared w2 */
    const int o = blockIdx.x * 16 + r;
    const int sbase = kpart * NSW;
    /* the shared w2 stream of this lane (FP8, one 512-slice per wave) */
    ApusWLane wsh{};
    if constexpr (SH) {
        ApusGemmEnt ent;
        ent.w = args.shw[1]; ent.ws = args.shws[1];
        wsh = apus_wlane<APUS_W_FP8>(ent, args.sh_tiled, o, lane, K);
    }
    for (int t = 0; t < args.acc_s; ++t) {
        const int p0 = t * NP;
        /* Load order: the token's expert ids (all in flight together), then
         * the weight ring, then the h rows. Loads behind a branch make the
         * compiler drain every load in flight, so nothing here is
         * conditional, and the weight stream starts one memory round trip
         * after the launch instead of after the h rows and one round trip
         * per pair. */
        int ev[NP];
#pragma unroll
        for (int j = 0; j < NP; ++j) ev[j] = apus_gld<int>(args.pidx + p0 + j);
        bool okj[NP];
#pragma unroll
        for (int j = 0; j < NP; ++j) okj[j] = (unsigned)ev[j] < (unsigned)args.pE;
        /* one uniform branch for all pairs (slab arithmetic or pointer
         * tables), not one per pair */
        ApusGemmEnt ents[NPG];
        if (args.pbase) {
#pragma unroll
            for (int jl = 0; jl < NPG; ++jl) {
                const uint8_t *b = args.pbase + (size_t)(okj[jb + jl] ? ev[jb + jl] : 0) * args.pstride;
                ents[jl].w = b + args.pwoff[0];
                ents[jl].ws = b + args.psoff[0];
            }
        } else {
#pragma unroll
            for (int jl = 0; jl < NPG; ++jl) {
                const int e = okj[jb + jl] ? ev[jb + jl] : 0;
                ents[jl].w = apus_gld<const uint8_t *>(args.pw[0] + e);
                ents[jl].ws = apus_gld<const uint8_t *>(args.pws[0] + e);
            }
        }
        ApusWLane wl[NPG];
#pragma unroll
        for (int jl = 0; jl < NPG; ++jl) wl[jl] = apus_wlane<APUS_W_FP4>(ents[jl], args.wtiled, o, lane, K);
        ApusBFrag<APUS_W_FP4> ring[PD];
#pragma unroll
        for (int u = 0; u < PD; ++u) apus_load_b_full<APUS_W_FP4>(ring[u], wl[u / NSW], sbase + u % NSW);
        /* A operands straight from the quantised h rows: lane (r, g) holds
         * row r's codes for its K sub-blocks (pair r, or the shared h as row
         * NP); an MFMA for pair j masks every row but j. Rows that feed no
         * MFMA read row p0 and get a finite scale (their codes are masked). */
        const bool arow = r < NR;
        const int hr = r < NP ? p0 + r : args.npairs + t;
        const int hrl = arow ? hr : p0;
        const uint8_t *ab = args.hq + (size_t)hrl * K + g * 16;
        uint4 av[NSW][4][2];
        unsigned asv[NSW];
#pragma unroll
        for (int si = 0; si < NSW; ++si) {
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const int q = (sbase + si) * 4 + st;
                av[si][st][0] = apus_gld<uint4>(ab + q * 128);
                av[si][st][1] = apus_gld<uint4>(ab + q * 128 + 64);
            }
            const unsigned sv = apus_gld<unsigned>(args.hqs + (size_t)hrl * NQ + (sbase + si) * 4);
            asv[si] = arow ? sv : 0x7f7f7f7fu;
        }
        ApusBFrag<APUS_W_FP8> fsh;
        if (shg) apus_load_b_full<APUS_W_FP8>(fsh, wsh, sbase);
        apus_v4f acc[NPG];
#pragma unroll
        for (int j = 0; j < NPG; ++j) acc[j] = apus_v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int stp = 0; stp < STEPS; ++stp) {
            const int jl = stp / NSW, j = jb + jl, si = stp % NSW;
            ApusBFrag<APUS_W_FP4> &cur = ring[stp % PD];
            const int z = r == j ? -1 : 0;
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const uint4 a0 = av[si][st][0], a1 = av[si][st][1];
                const apus_v8i a = apus_v8i{(int)a0.x & z, (int)a0.y & z, (int)a0.z & z, (int)a0.w & z,
                                            (int)a1.x & z, (int)a1.y & z, (int)a1.z & z, (int)a1.w & z};
                const apus_v4u w = cur.w[st][0];
                const apus_v8i b = apus_v8i{(int)w.x, (int)w.y, (int)w.z, (int)w.w, 0, 0, 0, 0};
                const int sa = (int)((asv[si] >> (8 * st)) & 0xffu);
                const int sb = (int)((cur.s[st] >> (8 * g)) & 0xffu);
                acc[jl] = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E2M1, 0, 0>(a, b, acc[jl], sa, sb);
            }
            if (stp + PD < STEPS)
                apus_load_b_full<APUS_W_FP4>(cur, wl[(stp + PD) / NSW], sbase + (stp + PD) % NSW);
        }
        apus_v4f accs = {0.f, 0.f, 0.f, 0.f};
        if (shg) {
            const int z = r == NP ? -1 : 0;
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const uint4 a0 = av[0][st][0], a1 = av[0][st][1];
                const apus_v8i a = apus_v8i{(int)a0.x & z, (int)a0.y & z, (int)a0.z & z, (int)a0.w & z,
                                            (int)a1.x & z, (int)a1.y & z, (int)a1.z & z, (int)a1.w & z};
                const apus_v4u w0 = fsh.w[st][0], w1 = fsh.w[st][1];
                const apus_v8i b = apus_v8i{(int)w0.x, (int)w0.y, (int)w0.z, (int)w0.w,
                                            (int)w1.x, (int)w1.y, (int)w1.z, (int)w1.w};
                const int sa = (int)((asv[0] >> (8 * st)) & 0xffu);
                accs = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E4M3, 0, 0>(a, b, accs, sa,
                                                                            (int)fsh.s[st]);
            }
        }
        apus_lds_barrier();                 /* the previous token's lred readers are done */
        /* pair j's result sits in D[j][r]: lane (g = j / 4, r), element j % 4.
         * Every lane stores (the reader picks the right lane): a store under a
         * lane-dependent condition would be the only consumer of the MFMA
         * results, and the compiler then sinks the MFMAs into the narrowed-EXEC
         * region, where a matrix instruction does not see the inactive lanes */
#pragma unroll
        for (int jl = 0; jl < NPG; ++jl) lred[kpart][jb + jl][lane] = acc[jl][(jb + jl) & 3];
        if (shg) lred[kpart][NP][lane] = accs[NP & 3];
        __syncthreads();
        if (threadIdx.x < 16) {
            float y = 0.0f;
#pragma unroll
            for (int j = 0; j < NP; ++j) {
                const int src = (j >> 2) * 16 + threadIdx.x;
                float eo = lred[0][j][src];
#pragma unroll
                for (int kp = 1; kp < KS; ++kp) eo += lred[kp][j][src];
                eo = okj[j] ? apus_bf16_rne(eo) : 0.0f;
                y = __fadd_rn(y, __fmul_rn(apus_gld<float>(args.acc_w + p0 + j), eo));
            }
            const size_t oo = (size_t)t * args.ldo + blockIdx.x * 16 + threadIdx.x;
            apus_gst<float>(args.acc_y + oo, y);
            if constexpr (SH) {
                const int src = (NP >> 2) * 16 + threadIdx.x;
                float sh = lred[0][NP][src];
#pragma unroll
                for (int kp = 1; kp < KS; ++kp) sh += lred[kp][NP][src];
                sh = apus_bf16_rne(sh);
                apus_gst<float>(args.sh_out + oo, sh);
                apus_gst<float>(args.add_out + oo, apus_bf16_rne(y + sh));
            } else if (args.add_out) {
                apus_gst<float>(args.add_out + oo, apus_bf16_rne(y + apus_gld<float>(args.add_src + oo)));
            }
        }
    }
}

hipError_t apus_launch_moe_pair13(const ApusGemmArgs *a, int npairs, hipStream_t st) {
    if (npairs <= 0) return hipSuccess;
    if ((a->K != 2048 && a->K != 4096) || a->O % 32 || a->npairs != npairs) return hipErrorInvalidValue;
    const bool sh = a->shw[0] != nullptr;
    if (sh && (a->acc_s <= 0 || a->O % 128)) return hipErrorInvalidValue;
    if (a->rsp && (a->rE <= 0 || a->rE > 1024 || a->adiv > 16 || a->adiv > a->rE || !a->ridx ||
                   !a->rwgt || (!a->rt2e && !a->rsel) || (a->rt2e && !a->rids)))
        return hipErrorInvalidValue;
    if (a->rdout && (!a->rdw || !a->rdws || a->acc_s <= 0 || a->O % 128)) return hipErrorInvalidValue;
    const int rows = npairs + (sh ? a->acc_s : 0) + (a->rdout ? a->acc_s : 0);
    /* 128-column workgroups (16 waves) quantise h themselves; 32-column ones
     * hand it over through counters. The wide ones win once they give at
     * least one workgroup per CU (4 tokens of top-6: 3.7 us less per
     * layer), the narrow ones below that (one token: 5 us less).
     * APUS_HIP_PAIR13_WIDE = 0 / 1 forces one. */
    static const int force = [] {
        const char *v = getenv("APUS_HIP_PAIR13_WIDE");
        return v ? atoi(v) : -1;
    }();
    const bool wide = force >= 0 ? force != 0 : (size_t)(a->O / 128) * rows >= 256;
#define APUS_P13(NS, SH, T) hipLaunchKernelGGL((apus_moe_pair13_kernel<NS, SH, T>), \
        dim3(a->O / (16 * T), rows), dim3(128 * T), 0, st, *a)
    if (wide && a->hq && a->O % 128 == 0 && !a->zero) {
        if (a->K == 4096) { if (sh) APUS_P13(8, true, 8); else APUS_P13(8, false, 8); }
        else              { if (sh) APUS_P13(4, true, 8); else APUS_P13(4, false, 8); }
    } else {
        if (a->K == 4096) { if (sh) APUS_P13(8, true, 2); else APUS_P13(8, false, 2); }
        else              { if (sh) APUS_P13(4, true, 2); else APUS_P13(4, false, 2); }
    }
#undef APUS_P13
    return hipGetLastError();
}

hipError_t apus_launch_moe_pair2(const ApusGemmArgs *a, hipStream_t st) {
    if (a->acc_s <= 0) return hipSuccess;
    if ((a->K != 2048 && a->K != 4096) || a->O % 16 || (a->acc_topk != 6 && a->acc_topk != 8) ||
        !a->hq || !a->hqs || a->npairs < a->acc_s * a->acc_topk)
        return hipErrorInvalidValue;
    const bool sh = a->shw[1] != nullptr;
    /* the fused shared w2 needs K = 2048 (one 512-slice per wave), its
     * outputs and the sum's destination */
    if (sh && (a->K != 2048 || a->O % 128 || !a->sh_out || !a->add_out ||
               a->npairs != a->acc_s * a->acc_topk))
        return hipErrorInvalidValue;
#ifndef APUS_PAIR2_GROUPS
#define APUS_PAIR2_GROUPS 1
#endif
    dim3 grid(a->O / 16), block(256 * APUS_PAIR2_GROUPS);
#define APUS_P2(NS, NP, SH) hipLaunchKernelGGL((apus_moe_pair2_kernel<NS, NP, SH, APUS_PAIR2_GROUPS>), grid, block, 0, st, *a)
    if (a->K == 4096) {
        if (a->acc_topk == 6) APUS_P2(8, 6, false);
        else                  APUS_P2(8, 8, false);
    } else if (sh) {
        if (a->acc_topk == 6) APUS_P2(4, 6, true);
        else                  APUS_P2(4, 8, true);
    } else {
        if (a->acc_topk == 6) APUS_P2(4, 6, false);
        else                  APUS_P2(4, 8, false);
    }
#undef APUS_P2
    return hipGetLastError();
}

/*
 * One-token MoE layer in ONE launch (apus_moe_layer1_kernel): the work of
 * apus_moe_pair13 (w1/w3 of the 6 routed pairs, optionally a dense FP8
 * [4096, 4096] linear of the same x riding along) and of apus_moe_pair2 (w2
 * and y = sum_j wgt * bf16(eo_j)) for dim 4096, inter 2048, topk 6, with a
 * barrier between the phases instead of a kernel boundary.
 *
 * 256 workgroups of 8 waves, one per CU (the launcher checks that 256 fit at
 * once; a barrier over workgroups that are not all resident would wait for
 * ever, so the wait is also bounded). Workgroup b:
 *  - phase 1 (b < 192): two pair13 units (32 inter rows of one pair each,
 *    one per 4-wave half: units 2b and 2b + 1, unit u = pair u / 64, column
 *    block u % 64), each computed exactly as apus_moe_pair13 with TILES = 2
 *    (same MFMA chain over K, same h hand-off through the per-group
 *    counters and quantisation by the group's last unit), then the
 *    workgroup arrives at the barrier; b >= 192 arrive at once;
 *  - after arriving, issues the loads of its rider slice, if any, then of
 *    its w2 share: 16 columns of dim for all 6 pairs, 102 KB, held in
 *    registers (wave group i takes pairs 3i..3i+2, its 4 waves the K
 *    quarters, as apus_moe_pair2 with G = 2); these bytes stream during the
 *    hand-off and barrier latency, not in front of the phase-1 refills;
 *  - the rider, if any: the 64 workgroups without pair units multiply 4
 *    16-row tiles of the rider's weight each (wave w: K slice w), 16.8 MB
 *    that do not depend on h;
 *    out = bf16(sum of the 8 slice chains in order), which may differ from
 *    the two-launch path's single K chain by fp32 rounding;
 *  - waits at the barrier (apus_l1_arrive / apus_l1_wait);
 *  - phase 2: the w2 MFMAs on the registers loaded at the arrival, the K
 *    quarters met in LDS, y written (and add_out = bf16(y + add_src)).
 * y and the h codes are bit-identical to the two-launch path.
 */
/* Phase barrier words (device memory, zero when allocated): the top arrival
 * counter (left zero), 8 release words (one per group of workgroups b & 7),
 * a fault counter and 8 group arrival counters (left zero), each 1 KB from
 * the next. */
#define APUS_L1_COUNT 0
#define APUS_L1_GEN(i) ((1 + (i)) * 256)
#define APUS_L1_FAULT (9 * 256)
#define APUS_L1_GROUP(i) ((10 + (i)) * 256)
#define APUS_L1_BAR_WORDS (18 * 256)
struct ApusLayerBar {
    unsigned *w;
    unsigned *hflag;     /* host-visible word set to 1 when a wait gives up (or null) */
    unsigned spin_lim;   /* polls of the release word before a wait gives up */
};


/* Phase barrier of the one-launch layer. Every workgroup arrives once, after
 * its phase-1 duties (its units' h stores and, for the unit that completes
 * an h group, the group's codes, all complete): first at the counter of its
 * group b & 7 (32 arrivals), and the last of a group at the top counter (8
 * arrivals); the 8th top arrival resets it and bumps the 8 release words (one
 * per group). Same-address atomics serialise: one counter taking every
 * arrival (the 96 group-completing units and the 64 workgroups without
 * units) was measured against this two-level count in a microbenchmark of
 * 256 simultaneous arrivals: release seen after 3.8 against 1.8 us.
 * Every workgroup reads its release word at its start, before its own
 * arrival, which the release needs. The release words spread the polling:
 * one word polled by all 256 workgroups, which the arrivals also hit,
 * measured 3.4 us slower per launch.
 * The barrier orders nothing in memory itself (no release / acquire fences:
 * at device scope those write back and invalidate a whole XCD's L2,
 * measured at ~3 us per launch here): the data that crosses it (the h
 * codes) is written with device-coherent stores that have completed
 * (s_waitcnt) before the writer's workgroup arrives, and read only after it,
 * by loads that cannot hit stale cache lines: no workgroup reads those lines
 * before the barrier in a launch, and every launch starts with invalidated
 * caches (HIP's stream order: a kernel, a graph node included, sees every
 * earlier kernel's writes, so the non-coherent L1 / L2 are invalidated at
 * its start). Reading them with device-coherent loads instead (two 8-byte
 * sc1 loads per 16 bytes) measured 975-991 against 1019-1030 tok/s at
 * config 4 on one box: those loads skip L2 on the barrier's critical path. */
#define APUS_L1_WGS 256u
__device__ __forceinline__ void apus_l1_arrive(const ApusLayerBar &bar) {
    unsigned *gc = bar.w + APUS_L1_GROUP(blockIdx.x & 7u);
    if (__hip_atomic_fetch_add(gc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != APUS_L1_WGS / 8u - 1u) return;
    __hip_atomic_store(gc, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    unsigned *cnt = bar.w + APUS_L1_COUNT;
    if (__hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 7u) return;
    __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
    for (unsigned i = 0; i < 8; ++i)
        __hip_atomic_fetch_add(bar.w + APUS_L1_GEN(i), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* Returns true in every thread when this workgroup gave up waiting: the
 * release was not seen within bar.spin_lim polls (about a second at the
 * default 2^23; 0 gives up at once). The fault counter is bumped and the
 * host-visible flag set, and the caller poisons its outputs with NaN. */
__device__ __forceinline__ bool apus_l1_wait(const ApusLayerBar &bar, unsigned g0, int &tmo) {
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned *genp = bar.w + APUS_L1_GEN(blockIdx.x & 7u);
        unsigned spins = 0;
        bool gave_up = false;
        while (__hip_atomic_load(genp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == g0) {
            if (spins++ >= bar.spin_lim) { gave_up = true; break; }
            __builtin_amdgcn_s_sleep(1);
        }
        if (gave_up) {
            __hip_atomic_fetch_add(bar.w + APUS_L1_FAULT, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (bar.hflag) __hip_atomic_store(bar.hflag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
        tmo = gave_up;
    }
    __syncthreads();
    return tmo != 0;
}

/* phase-1 MFMA chain of one wave: row 0 of A is x (codes in LDS), the tile's
 * 16 weight rows stream through `ring` (issued by the caller), as in
 * apus_pair13_body */
template <int WF, int NS, int PD, bool SC = true>
__device__ __forceinline__ apus_v4f apus_layer1_chain(ApusBFrag<WF> (&ring)[PD], const ApusWLane &wl,
                                                      const uint8_t *lcodes, const uint8_t *lsc,
                                                      int r, int g, int s0,
                                                      const apus_v4u *scs = nullptr) {
    const int z = r == 0 ? -1 : 0;
    const uint8_t *arow = lcodes + g * 16;
    apus_v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        ApusBFrag<WF> &cur = ring[s % PD];
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const int q = (s0 + s) * 4 + st;
            const uint4 a0 = *reinterpret_cast<const uint4 *>(arow + q * 128);
            const uint4 a1 = *reinterpret_cast<const uint4 *>(arow + q * 128 + 64);
            const apus_v8i a = apus_v8i{(int)a0.x & z, (int)a0.y & z, (int)a0.z & z, (int)a0.w & z,
                                        (int)a1.x & z, (int)a1.y & z, (int)a1.z & z, (int)a1.w & z};
            if constexpr (WF == APUS_W_FP4) {
                const apus_v4u w = cur.w[st][0];
                const apus_v8i b = apus_v8i{(int)w.x, (int)w.y, (int)w.z, (int)w.w, 0, 0, 0, 0};
                const int sb = (int)(((SC ? cur.s[st] : scs[s][st]) >> (8 * g)) & 0xffu);
                acc = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E2M1, 0, 0>(a, b, acc, (int)lsc[q], sb);
            } else {
                const apus_v4u w0 = cur.w[st][0], w1 = cur.w[st][1];
                const apus_v8i b = apus_v8i{(int)w0.x, (int)w0.y, (int)w0.z, (int)w0.w,
                                            (int)w1.x, (int)w1.y, (int)w1.z, (int)w1.w};
                acc = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E4M3, 0, 0>(a, b, acc, (int)lsc[q],
                                                                           (int)cur.s[st]);
            }
        }
        if (s + PD < NS) apus_load_b_full<WF, SC>(cur, wl, s0 + s + PD);
    }
    return acc;
}

/* shared memory of apus_moe_layer1_kernel */
struct ApusLayer1Lds {
    uint8_t codes[4096 + 32];
    uint8_t sc[32];
    float gu[2][2][2][64];                    /* [half][mat][tile][lane] */
    float red[4][6][64];                      /* [K quarter][pair][lane] */
    float rr[4][8][64];                       /* rider partial sums [tile][wave][lane] */
    int last[2];
    int tmo;                                  /* the barrier wait gave up */
};


/* The workgroup's whole program for one role (ROLE 0: two pair units; 2: no
 * pair units), so that each role's registers are allocated on their own. */
template <int ROLE>
__device__ __forceinline__ void apus_layer1_role(const ApusGemmArgs &a1, const ApusGemmArgs &a2,
                                                 const ApusLayerBar &bar, ApusLayer1Lds &L) {
    constexpr int K1 = 4096, NS1 = 8, O1 = 2048;
#ifndef APUS_L1_PD
#define APUS_L1_PD 3
#endif
    constexpr int K2 = 2048, NQ2 = 16, NP = 6, NPG = 3, KS = 4, PD1 = APUS_L1_PD;
    const int b = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int half = wave >> 2, w4 = wave & 3;
    const int r = lane & 15, g = lane >> 4;
    const bool rd = a1.rdout != nullptr;

    /* this workgroup's barrier release word, read before anything else
     * (every lane reads the same word: no branch around the load) */
    const unsigned g0 = __hip_atomic_load(bar.w + APUS_L1_GEN(blockIdx.x & 7u), __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
    /* x row (one token): its loads go out first */
    ApusStageRaw<APUS_A_F32> raw;
    apus_stage_load<K1, APUS_A_F32>(a1, nullptr, 0, 0, 1, 0, raw);
    /* the token's expert ids, all in flight together */
    int ev[NP];
#pragma unroll
    for (int j = 0; j < NP; ++j) ev[j] = apus_gld<int>(a1.pidx + j);
    bool okj[NP];
#pragma unroll
    for (int j = 0; j < NP; ++j) okj[j] = (unsigned)ev[j] < (unsigned)a1.pE;
    /* the routing weights (inputs of the launch) */
    float wj[NP];
#pragma unroll
    for (int j = 0; j < NP; ++j) wj[j] = apus_gld<float>(a2.acc_w + j);

    /* phase-1 unit of this half (ROLE 0) */
    const int mat = w4 & 1, tile = w4 >> 1;
    const int u = 2 * b + half, p = u >> 6, cb = u & 63;
    const int o1 = cb * 32 + tile * 16 + r;
    int ep = ev[0];
#pragma unroll
    for (int j = 1; j < NP; ++j) ep = p == j ? ev[j] : ep;
    const bool okp = (unsigned)ep < (unsigned)a1.pE;
    /* Every weight pointer first (one uniform branch: slab arithmetic or
     * pointer tables), then the phase-1 ring (the w2 share follows the
     * arrival). A load behind a branch, or a wait
     * for a pointer issued after weight loads, would make the compiler
     * drain the loads in flight. Weights are MFMA-tiled (the launcher
     * checks). */
    const int jb = half * NPG, o2 = b * 16 + r;
    ApusGemmEnt ent1, ents2[NPG];
    if (a1.pbase) {
        if constexpr (ROLE == 0) {
            const uint8_t *base = a1.pbase + (size_t)(okp ? ep : 0) * a1.pstride;
            ent1.w = base + (mat ? a1.pwoff[1] : a1.pwoff[0]);
            ent1.ws = base + (mat ? a1.psoff[1] : a1.psoff[0]);
        }
#pragma unroll
        for (int jl = 0; jl < NPG; ++jl) {
            const uint8_t *base = a2.pbase + (size_t)(okj[jb + jl] ? ev[jb + jl] : 0) * a2.pstride;
            ents2[jl].w = base + a2.pwoff[0];
            ents2[jl].ws = base + a2.psoff[0];
        }
    } else {
        if constexpr (ROLE == 0) {
            const int e = okp ? ep : 0;
            ent1.w = apus_gld<const uint8_t *>((mat ? a1.pw[1] : a1.pw[0]) + e);
            ent1.ws = apus_gld<const uint8_t *>((mat ? a1.pws[1] : a1.pws[0]) + e);
        }
#pragma unroll
        for (int jl = 0; jl < NPG; ++jl) {
            const int e = okj[jb + jl] ? ev[jb + jl] : 0;
            ents2[jl].w = apus_gld<const uint8_t *>(a2.pw[0] + e);
            ents2[jl].ws = apus_gld<const uint8_t *>(a2.pws[0] + e);
        }
    }
    ApusBFrag<APUS_W_FP4> ring1[PD1];
    ApusWLane wl1{};
    /* the group scales of the whole phase-1 stream in one burst ahead of
     * its ring (as the few-row schedule) */
    apus_v4u scs1[ROLE == 0 ? NS1 : 1];
    if constexpr (ROLE == 0) {
        wl1 = apus_wlane<APUS_W_FP4>(ent1, true, o1, lane, K1);
#pragma unroll
        for (int v = 0; v < NS1; ++v) scs1[v] = apus_gld<apus_v4u>(wl1.s + (size_t)v * wl1.ss);
#pragma unroll
        for (int v = 0; v < PD1; ++v) apus_load_b_full<APUS_W_FP4, false>(ring1[v], wl1, v);
    }
    ApusBFrag<APUS_W_FP4> ring2[NPG];
    /* the rider's rows of this workgroup: RT 16-row tiles of its [4096, 4096]
     * weight from tile rt0, wave w taking the 512-slice w of K (loaded after
     * the workgroup's arrival, below). With APUS_L1_RIDER2 the 64
     * workgroups without pair units take all 256 tiles (4 each), so that
     * the pair workgroups (256 KB of phase-1 weights each) stream only their
     * w2 share after arriving (config 4 +0.3 to +1.6 % in five same-box
     * pairs, e.g. 1030 against 1014 tok/s); else every workgroup takes tile
     * b. The tiles' sums are the same chains either way. */
#ifndef APUS_L1_RIDER2
#define APUS_L1_RIDER2 1
#endif
    constexpr int RT = APUS_L1_RIDER2 ? (ROLE == 2 ? 4 : 0) : 1;
    const int rt0 = APUS_L1_RIDER2 ? (b - 192) * 4 : b;
    ApusWLane wlr[RT > 0 ? RT : 1];
    if (rd) {
        ApusGemmEnt er;
        er.w = a1.rdw; er.ws = a1.rdws;
#pragma unroll
        for (int t = 0; t < RT; ++t) wlr[t] = apus_wlane<APUS_W_FP8>(er, true, (rt0 + t) * 16 + r, lane, K1);
    }

    apus_stage_quant<K1, APUS_A_F32>(a1, raw, L.codes, L.sc);
    apus_lds_barrier();
    /* ---- phase 1 ---- */
    if constexpr (ROLE == 0) {
        const apus_v4f acc = apus_layer1_chain<APUS_W_FP4, NS1, PD1, false>(ring1, wl1, L.codes, L.sc, r, g, 0, scs1);
        /* every lane stores its element (see apus_pair13_body) */
        L.gu[half][mat][tile][lane] = apus_bf16_rne(acc[0]);
        __syncthreads();
        const int ht = threadIdx.x & 255;            /* thread within the half */
        float *hdst = a1.pout[0] + (size_t)p * O1;
        if (ht < 32) {
            const int t = ht >> 4, rr = ht & 15;
            const float h = okp ? apus_swiglu_h(L.gu[half][0][t][rr], L.gu[half][1][t][rr], a1.limit) : 0.0f;
            __hip_atomic_store(hdst + cb * 32 + t * 16 + rr, h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        /* the four units of a 128-column group take tickets; the last
         * quantises the group (as apus_pair13_body) and arrives */
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        constexpr int G = O1 >> 7;
        const int gq = cb >> 2;
        unsigned *tk = a1.hq_tk + (size_t)p * G + gq;
        if (ht == 0)
            L.last[half] = __hip_atomic_fetch_add(tk, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 3u;
        __syncthreads();
        if (L.last[half] && ht < 8) {
            const float *src = hdst + gq * 128 + ht * 16;
            float v[16];
#pragma unroll
            for (int i = 0; i < 16; ++i)
                v[i] = apus_bf16_rne(__hip_atomic_load(src + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
            float m = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) m = fmaxf(m, fabsf(v[i]));
            m = fmaxf(m, __shfl_xor(m, 1, 64));
            m = fmaxf(m, __shfl_xor(m, 2, 64));
            m = fmaxf(m, __shfl_xor(m, 4, 64));
            const uint32_t e8 = apus_act_scale_exp(m);
            const float inv = apus_inv_pow2_from_exp(e8);
            uint32_t q4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                q4[i] = apus_e4m3_pack4_hw(v[4 * i] * inv, v[4 * i + 1] * inv, v[4 * i + 2] * inv,
                                           v[4 * i + 3] * inv);
            /* device-coherent: the w2 phase on other XCDs reads them */
            unsigned *hw = reinterpret_cast<unsigned *>(a1.hq + (size_t)p * O1 + gq * 128 + ht * 16);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                __hip_atomic_store(hw + i, q4[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (ht == 0) {
                __hip_atomic_store(a1.hqs + (size_t)p * G + gq, (uint8_t)e8, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(tk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   /* complete before arriving */
        }
        /* both halves' hand-off duties are done (the completers' stores have
         * completed above): the workgroup arrives once */
        apus_lds_barrier();
        if (threadIdx.x == 0) apus_l1_arrive(bar);
    } else {
        /* workgroups without pair units arrive at once */
        if (threadIdx.x == 0) apus_l1_arrive(bar);
    }
    /* The rider (a dense FP8 linear of x, independent of h) streams while
     * the h hand-off and the barrier run: a workgroup loads its slices only
     * after every wait that precedes its arrival (a wait counts every load
     * issued before it; issuing them right after the phase-1 chain instead,
     * with LDS-only barriers in the hand-off, and at the start in the
     * workgroups without pair units, measured 5 % slower per layer); the
     * MFMAs run before the wait. */
    ApusBFrag<APUS_W_FP8> fr[RT > 0 ? RT : 1];
    if (rd) {
#pragma unroll
        for (int t = 0; t < RT; ++t) apus_load_b_full<APUS_W_FP8>(fr[t], wlr[t], wave);
    }
    /* the w2 share (wave group `half` takes pairs 3 half .. 3 half + 2, wave
     * w4 the K quarter w4, one 512-slice each), issued after the arrival:
     * issued with the phase-1 ring, its bytes sat in front of the chain's
     * refills (loads complete in order) while the hand-off and barrier
     * window carried only the rider */
#pragma unroll
    for (int jl = 0; jl < NPG; ++jl)
        apus_load_b_full<APUS_W_FP4>(ring2[jl], apus_wlane<APUS_W_FP4>(ents2[jl], true, o2, lane, K2), w4);
    if (rd) {
        const int z = r == 0 ? -1 : 0;
        const uint8_t *arow = L.codes + g * 16;
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            apus_v4f accr = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const int q = wave * 4 + st;
                const uint4 x0 = *reinterpret_cast<const uint4 *>(arow + q * 128);
                const uint4 x1 = *reinterpret_cast<const uint4 *>(arow + q * 128 + 64);
                const apus_v8i a = apus_v8i{(int)x0.x & z, (int)x0.y & z, (int)x0.z & z, (int)x0.w & z,
                                            (int)x1.x & z, (int)x1.y & z, (int)x1.z & z, (int)x1.w & z};
                const apus_v4u w0 = fr[t].w[st][0], w1 = fr[t].w[st][1];
                const apus_v8i bb = apus_v8i{(int)w0.x, (int)w0.y, (int)w0.z, (int)w0.w,
                                             (int)w1.x, (int)w1.y, (int)w1.z, (int)w1.w};
                accr = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E4M3, 0, 0>(a, bb, accr, (int)L.sc[q],
                                                                           (int)fr[t].s[st]);
            }
            L.rr[t][wave][lane] = accr[0];            /* lane (g 0, r): weight row 16 (rt0 + t) + r */
        }
    }
    /* a workgroup that gave up waiting may read h codes not yet written:
     * its y (and add_out) columns are written as NaN */
    const bool tmo = apus_l1_wait(bar, g0, L.tmo);

    /* ---- phase 2 (as apus_moe_pair2_kernel, G = 2, one token) ---- */
    /* the h codes and scale bytes (see apus_l1_arrive for why plain
     * loads see them) */
    const bool arow = r < NP;
    const uint8_t *ab = a2.hq + (size_t)(arow ? r : 0) * K2 + g * 16;
    apus_v8i av[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
        const int q = w4 * 4 + st;
        const uint4 x0 = apus_gld<uint4>(ab + q * 128), x1 = apus_gld<uint4>(ab + q * 128 + 64);
        av[st] = apus_v8i{(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
    }
    const unsigned sv = apus_gld<unsigned>(a2.hqs + (size_t)(arow ? r : 0) * NQ2 + w4 * 4);
    const unsigned asv = arow ? sv : 0x7f7f7f7fu;
    apus_v4f acc2[NPG];
#pragma unroll
    for (int jl = 0; jl < NPG; ++jl) {
        const int j = jb + jl;
        const int z = r == j ? -1 : 0;
        acc2[jl] = apus_v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const apus_v8i a = av[st] & apus_v8i{z, z, z, z, z, z, z, z};
            const apus_v4u w = ring2[jl].w[st][0];
            const apus_v8i bb = apus_v8i{(int)w.x, (int)w.y, (int)w.z, (int)w.w, 0, 0, 0, 0};
            const int sa = (int)((asv >> (8 * st)) & 0xffu);
            const int sb = (int)((ring2[jl].s[st] >> (8 * g)) & 0xffu);
            acc2[jl] = apus_mfma_scaled<APUS_FMT_E4M3, APUS_FMT_E2M1, 0, 0>(a, bb, acc2[jl], sa, sb);
        }
    }
#pragma unroll
    for (int jl = 0; jl < NPG; ++jl) L.red[w4][jb + jl][lane] = acc2[jl][(jb + jl) & 3];
    __syncthreads();
    if (threadIdx.x < 16) {
        float y = 0.0f;
#pragma unroll
        for (int j = 0; j < NP; ++j) {
            const int src = (j >> 2) * 16 + threadIdx.x;
            float eo = L.red[0][j][src];
#pragma unroll
            for (int kp = 1; kp < KS; ++kp) eo += L.red[kp][j][src];
            eo = okj[j] ? apus_bf16_rne(eo) : 0.0f;
            y = __fadd_rn(y, __fmul_rn(wj[j], eo));
        }
        if (tmo) y = __builtin_nanf("");
        const size_t oo = (size_t)b * 16 + threadIdx.x;
        apus_gst<float>(a2.acc_y + oo, y);
        if (a2.add_out)
            apus_gst<float>(a2.add_out + oo, apus_bf16_rne(y + apus_gld<float>(a2.add_src + oo)));
    } else if (rd && RT > 0 && threadIdx.x < 16 + 16 * RT) {
        /* the rider's row 16 (rt0 + t) + i: bf16 of the 8 K-slice sums in
         * order */
        const int t = (threadIdx.x - 16) >> 4, i = (threadIdx.x - 16) & 15;
        float v = L.rr[t][0][i];
#pragma unroll
        for (int w = 1; w < 8; ++w) v += L.rr[t][w][i];
        apus_gst<float>(a1.rdout + (size_t)(rt0 + t) * 16 + i, apus_bf16_rne(v));
    }
}

__global__ __launch_bounds__(512) void apus_moe_layer1_kernel(ApusGemmArgs a1, ApusGemmArgs a2,
                                                              ApusLayerBar bar) {
    __shared__ __align__(16) ApusLayer1Lds L;
    if (blockIdx.x < 192)
        apus_layer1_role<0>(a1, a2, bar, L);
    else
        apus_layer1_role<2>(a1, a2, bar, L);
}

hipError_t apus_launch_moe_layer1(const ApusGemmArgs *a1, const ApusGemmArgs *a2, unsigned *bar,
                                  unsigned *hflag, unsigned spin_lim, hipStream_t st) {
    if (a1->K != 4096 || a1->O != 2048 || a1->npairs != 6 || a1->adiv != 6 || a1->acc_s != 1 ||
        !a1->wtiled || !a2->wtiled || (a1->rdout && !a1->rdtiled) || !a1->pbase != !a2->pbase ||
        a1->shw[0] || a1->rsp || a1->zero || !a1->hq || !a1->hqs || !a1->hq_tk || !a1->pidx ||
        a2->K != 2048 || a2->O != 4096 || a2->acc_topk != 6 || a2->acc_s != 1 || a2->shw[1] ||
        a2->hq != a1->hq || a2->hqs != a1->hqs || a2->pidx != a1->pidx || !bar ||
        (a1->rdout && (!a1->rdw || !a1->rdws)))
        return hipErrorInvalidValue;
    ApusLayerBar b{bar, hflag, spin_lim};
    hipLaunchKernelGGL(apus_moe_layer1_kernel, dim3(APUS_L1_WGS), dim3(512), 0, st, *a1, *a2, b);
    return hipGetLastError();
}

int apus_moe_layer1_bar_words() { return APUS_L1_BAR_WORDS; }
int apus_moe_layer1_fault_word() { return APUS_L1_FAULT; }

int apus_moe_layer1_fits() {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, apus_moe_layer1_kernel, 512, 0) != hipSuccess)
        return 0;
    return n;
}

namespace {

template <int WF, int R, int NS, int KS, int ASRC, bool FOLD = false>
void apus_launch_dec(const ApusGemmArgs &d, int n_ent, hipStream_t st) {
#ifndef APUS_DEC_PD_FP4
#define APUS_DEC_PD_FP4 3
#endif
/* the K-quarter-order launches (the routed w2, K = 2048: four slices per
 * wave) run a ring of two: 160 -> fewer VGPRs, 141.5 -> 137.5 us per launch
 * over configs 2 and 3 (rocprof, same box) */
#ifndef APUS_DEC_PD_FOLD
#define APUS_DEC_PD_FOLD 2
#endif
    constexpr int NSW = NS / KS, PDD = WF == APUS_W_FP4 ? (FOLD ? APUS_DEC_PD_FOLD : APUS_DEC_PD_FP4) : 2;
    constexpr int PD = PDD < NSW ? PDD : NSW;
    constexpr int K = NS * 512, NQ = NS * 4;
    const size_t lds = (((size_t)R * (K + 32) + (size_t)R * NQ + 15) & ~(size_t)15) +
                       (KS > 1 ? APUS_DEC_NT * sizeof(float) * 4 : 0);
    if (lds > 65536) {
        /* eight staged rows of K = 8192 need more than the default 64 KB */
        static const hipError_t attr = hipFuncSetAttribute(
            reinterpret_cast<const void *>(&apus_gemm_decode_kernel<WF, R, NS, PD, KS, ASRC, FOLD>),
            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        (void)attr;
    }
    dim3 gd(d.O / (16 * APUS_DEC_WAVES / KS), n_ent), bd(APUS_DEC_NT);
    hipLaunchKernelGGL((apus_gemm_decode_kernel<WF, R, NS, PD, KS, ASRC, FOLD>), gd, bd, lds, st, d);
}

/* the K split for K = 512 * NS: KS divides NS; single-row chunks always split
 * K (with one chunk per workgroup and whole-K waves the compiler hoists every
 * slice's weight loads and runs out of registers) */
template <int WF, int R, int NS, int ASRC>
void apus_launch_dec_ns(const ApusGemmArgs &d, int n_ent, int ks, hipStream_t st) {
    if constexpr (NS >= 4 && APUS_DEC_WAVES % 4 == 0) {
        if (ks == 4) { apus_launch_dec<WF, R, NS, 4, ASRC>(d, n_ent, st); return; }
    }
    if constexpr (R != 1) {
        if (ks == 1) {
            /* the K-quarter order with whole-K waves: MXFP4 expert GEMMs on
             * pre-quantised rows (the routed w2 in sorted order) */
            if constexpr (WF == APUS_W_FP4 && ASRC == APUS_A_CODES && NS % 4 == 0) {
                if (d.kchain == 4) { apus_launch_dec<WF, R, NS, 1, ASRC, true>(d, n_ent, st); return; }
            }
            apus_launch_dec<WF, R, NS, 1, ASRC>(d, n_ent, st);
            return;
        }
    }
    apus_launch_dec<WF, R, NS, 2, ASRC>(d, n_ent, st);
}

template <int WF, int R, int ASRC>
void apus_launch_dec_k(const ApusGemmArgs &d, int n_ent, int ks, hipStream_t st) {
    if constexpr (ASRC != APUS_A_SWIGLU) {
        if (d.K == 1024) { apus_launch_dec_ns<WF, R, 2, ASRC>(d, n_ent, ks, st); return; }
        if (d.K == 8192) { apus_launch_dec_ns<WF, R, 16, ASRC>(d, n_ent, ks, st); return; }
    }
    if (d.K == 4096) apus_launch_dec_ns<WF, R, 8, ASRC>(d, n_ent, ks, st);
    else             apus_launch_dec_ns<WF, R, 4, ASRC>(d, n_ent, ks, st);
}

/* waves per 16-row tile: the smallest K split that still gives about one
 * wave per SIMD (1024 on 256 CUs); measured on gfx950, whole-K waves stream
 * best once there are enough of them (12 x 2048-row GEMVs: KS 1 10.8 us, KS 2
 * 13.2 us) and small launches need the split (one 4096-row FP8 GEMV: KS 4
 * 6.3 us, KS 1 8.8 us). APUS_HIP_DEC_KS (1, 2, 4) overrides. */
/* the resident-activation prefill schedule for the routed w2
 * (APUS_HIP_PRE_RA=0 turns it off) */
bool apus_pre_ra_on() {
    static const bool on = [] {
        const char *e = getenv("APUS_HIP_PRE_RA");
        return !(e && atoi(e) == 0);
    }();
    return on;
}

/* the same for the one-chain launches (the routed w1/w3;
 * APUS_HIP_PRE_RA13=0 turns it off) */
bool apus_pre_ra_w13() {
    static const bool on = [] {
        const char *e = getenv("APUS_HIP_PRE_RA13");
        return !(e && atoi(e) == 0);
    }();
    return on;
}

/* the LDS many-row schedule for work-list launches (APUS_HIP_PRE_LDS=0
 * turns it off: the resident-activation or prefill schedule, identical
 * bits; 1, the default: one-chain launches only; 2: the K-quarter ones as
 * well) */
int apus_pre_lds_mode() {
    static const int m = [] {
        const char *e = getenv("APUS_HIP_PRE_LDS");
        return e ? atoi(e) : 1;
    }();
    return m;
}
bool apus_pre_lds_on() { return apus_pre_lds_mode() != 0; }

/* the narrow schedule for dense FP8 GEMMs of 9..64 rows (APUS_HIP_NARROW=0
 * turns it off: the tile schedules) */
bool apus_narrow_on() {
    static const bool on = [] {
        const char *e = getenv("APUS_HIP_NARROW");
        return !(e && atoi(e) == 0);
    }();
    return on;
}

/* the grouped GEMV for few-row grouped launches on tiled weights
 * (APUS_HIP_GRP=0 turns it off: the few-row schedule) */
bool apus_grp_on() {
    static const bool on = [] {
        const char *e = getenv("APUS_HIP_GRP");
        return !(e && atoi(e) == 0);
    }();
    return on;
}

/* the split-K GEMV for few-row dense FP8 / MXFP4 launches on tiled weights
 * (APUS_HIP_SPLIT=0 turns it off: the few-row schedule) */
bool apus_split_on() {
    static const bool on = [] {
        const char *e = getenv("APUS_HIP_SPLIT");
        return !(e && atoi(e) == 0);
    }();
    return on;
}

/* the LDS tile schedule for dense FP8 GEMMs (APUS_HIP_LDS_TILE=0 turns it
 * off: the register-ring tile schedule, identical bits) */
bool apus_lds_tile_on() {
    static const bool on = [] {
        const char *e = getenv("APUS_HIP_LDS_TILE");
        return !(e && atoi(e) == 0);
    }();
    return on;
}

int apus_dec_ks_env() {
    static const int forced = [] {
        const char *e = getenv("APUS_HIP_DEC_KS");
        const int v = e ? atoi(e) : 0;
        return (v == 1 || v == 2 || v == 4) ? v : 0;
    }();
    return forced;
}
bool apus_dec_ks_forced() { return apus_dec_ks_env() != 0; }

int apus_dec_ks(size_t row_tiles) {
    const int forced = apus_dec_ks_env();
    if (forced) return forced;
    return row_tiles >= 1024 ? 1 : row_tiles >= 512 ? 2 : 4;
}

}  // namespace

hipError_t apus_launch_gemm_few(int wfmt, const ApusGemmArgs *a, int n_ent, int rows,
                                int ks, hipStream_t st) {
    if (n_ent <= 0) return hipSuccess;
    if (!apus_fast_k(a->K) || a->O % 128 || (rows != 1 && rows != 8) ||
        (a->asrc == APUS_A_CODES && rows != 8) ||
        (a->asrc == APUS_A_SWIGLU && !apus_group_k(a->K)) ||
        (a->acc_y && (!a->pidx || a->nmat != 1 || !a->tickets)) || ks < 0 || ks > 4 || ks == 3)
        return hipErrorInvalidValue;
    /* two by-value entries share their activation rows (staged once, before
     * the entry lookup) */
    if (!a->ents && !a->pidx &&
        (n_ent > 2 || (n_ent == 2 && (a->ent1.a0 != a->ent0.a0 || a->ent1.arows != a->ent0.arows ||
                                      a->ent1.M != a->ent0.M))))
        return hipErrorInvalidValue;
    /* one dense FP8 / MXFP4 entry on tiled weights: the split-K GEMV
     * (unless a K split is forced) */
    if (n_ent == 1 && !ks && !a->kchain && (wfmt == APUS_W_FP8 || APUS_SPLIT_FP4) && a->wtiled && !a->ents &&
        !a->pidx &&
        !a->acc_y && !a->add_out && !a->items && !a->hq && !a->rdout && !a->zero && !a->ent0.arows &&
        !a->ent0.orows && a->ent0.M <= 8 && (a->asrc == APUS_A_CODES || a->asrc == APUS_A_F32) &&
        apus_split_on() && !apus_dec_ks_forced()) {
        if (wfmt == APUS_W_FP8) {
            if (a->asrc == APUS_A_CODES) apus_launch_split<APUS_W_FP8, APUS_A_CODES>(*a, st);
            else                         apus_launch_split<APUS_W_FP8, APUS_A_F32>(*a, st);
        } else {
            if (a->asrc == APUS_A_CODES) apus_launch_split<APUS_W_FP4, APUS_A_CODES>(*a, st);
            else                         apus_launch_split<APUS_W_FP4, APUS_A_F32>(*a, st);
        }
        return hipGetLastError();
    }
    if (!ks) ks = apus_dec_ks((size_t)n_ent * (a->O / 16));
    /* a required accumulation order (kchain) fixes the K split: one chain
     * needs whole-K waves; the K-quarter order takes whole-K waves (folded
     * per quarter) or one quarter per wave */
    if (a->kchain == 1) {
        if (rows == 1) return hipErrorInvalidValue;   /* single-row chunks always split K */
        ks = 1;
    } else if (a->kchain == 4) {
        if (a->K < 2048) return hipErrorInvalidValue;
        const bool fold = rows == 8 && a->asrc == APUS_A_CODES && wfmt == APUS_W_FP4;
        ks = (ks == 1 && fold) ? 1 : 4;
    } else if (a->kchain != 0) {
        return hipErrorInvalidValue;
    }
    const bool fp4 = wfmt == APUS_W_FP4;
    switch (a->asrc) {
    case APUS_A_CODES:
        if (fp4) apus_launch_dec_k<APUS_W_FP4, 8, APUS_A_CODES>(*a, n_ent, ks, st);
        else     apus_launch_dec_k<APUS_W_FP8, 8, APUS_A_CODES>(*a, n_ent, ks, st);
        break;
    case APUS_A_F32:
        if (rows == 1) {
            if (fp4) apus_launch_dec_k<APUS_W_FP4, 1, APUS_A_F32>(*a, n_ent, ks, st);
            else     apus_launch_dec_k<APUS_W_FP8, 1, APUS_A_F32>(*a, n_ent, ks, st);
        } else {
            if (fp4) apus_launch_dec_k<APUS_W_FP4, 8, APUS_A_F32>(*a, n_ent, ks, st);
            else     apus_launch_dec_k<APUS_W_FP8, 8, APUS_A_F32>(*a, n_ent, ks, st);
        }
        break;
    case APUS_A_SWIGLU:
        if (rows == 1) {
            if (fp4) apus_launch_dec_k<APUS_W_FP4, 1, APUS_A_SWIGLU>(*a, n_ent, ks, st);
            else     apus_launch_dec_k<APUS_W_FP8, 1, APUS_A_SWIGLU>(*a, n_ent, ks, st);
        } else {
            if (fp4) apus_launch_dec_k<APUS_W_FP4, 8, APUS_A_SWIGLU>(*a, n_ent, ks, st);
            else     apus_launch_dec_k<APUS_W_FP8, 8, APUS_A_SWIGLU>(*a, n_ent, ks, st);
        }
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t apus_launch_gemm(int wfmt, const ApusGemmArgs *a, int n_ent,
                            hipStream_t st) {
    if (n_ent <= 0) return hipSuccess;
    const bool grouped = a->ents != nullptr;
    const size_t row_tiles = (size_t)n_ent * ((a->O + 15) / 16);
    constexpr int R = 8;
    if (a->items && (wfmt != APUS_W_FP4 || !grouped)) return hipErrorInvalidValue;
    if (a->wtiled) {
        /* tiled weights: only the decode, prefill and tile schedules read them */
        if (!(grouped ? apus_group_k(a->K) : apus_fast_k(a->K)) || a->O % 128)
            return hipErrorInvalidValue;
        if (!grouped && a->ent0.M <= R) {
            ApusGemmArgs d = *a;
            d.asrc = APUS_A_CODES;
            return apus_launch_gemm_few(wfmt, &d, 1, R, 0, st);
        }
    }
    /* grouped launches with K = 2048 or 4096: entries with at most 8 rows
     * take the decode schedule, larger ones the prefill schedule (two
     * launches over the same entry table, each skipping the other's entries) */
    if (grouped && (row_tiles >= 512 || (a->max_m > 0 && a->max_m <= R) || a->wtiled) &&
        apus_group_k(a->K) && a->O % 128 == 0) {
        const bool run_dec = !(a->min_m >= R);
        const bool run_pre = !(a->max_m > 0 && a->max_m <= R);
        /* few-row entries only, no required order, tiled weights: the
         * grouped GEMV */
        if (!run_pre && a->wtiled && !a->kchain && !a->pidx && !a->acc_y && !a->add_out && !a->items &&
            !a->zero && a->max_m > 0 && apus_grp_on()) {
            if (wfmt == APUS_W_FP4) apus_launch_grp<APUS_W_FP4>(*a, n_ent, st);
            else                    apus_launch_grp<APUS_W_FP8>(*a, n_ent, st);
            return hipGetLastError();
        }
        if (run_dec) {
            ApusGemmArgs d = *a;
            d.m_min = 0;
            d.m_max = R;
            d.asrc = APUS_A_CODES;
            const hipError_t e = apus_launch_gemm_few(wfmt, &d, n_ent, R, 0, st);
            if (e != hipSuccess) return e;
        }
        if (!run_pre) return hipGetLastError();
        ApusGemmArgs p = *a;
        p.m_min = R;
        p.m_max = 0;
        /* with a work list, n_ent counts its items */
        dim3 gp(a->O / (16 * APUS_PRE_WAVES), n_ent), bp(APUS_PRE_THREADS);
        if (wfmt == APUS_W_FP4) {
#ifndef APUS_PRE_PD4
#define APUS_PRE_PD4 2
#endif
            constexpr int TT4 = APUS_PREFILL_ROWS / 16;
            /* activations resident in LDS, NCB column blocks per workgroup
             * (work-list launches whose column blocks divide evenly) */
            const bool ra = a->items && TT4 == 4 && a->O % (128 * APUS_PRE_RA_NCB) == 0 && apus_pre_ra_on();
            /* one-chain work lists on tiled weights (the routed w1/w3): the
             * LDS many-row schedule (config 3 w1/w3 126 -> 121 us; for the
             * K-quarter w2 at K = 2048 it measured 89.5 against 78.9 us for
             * the resident-activation schedule, which keeps the chunk's
             * activations in LDS across four column blocks, so w2 stays
             * there; APUS_HIP_PRE_LDS=2 runs it for w2 as well) */
            if (a->items && a->wtiled && TT4 == 4 && apus_pre_lds_on()) {
                bool ok = false;
                if (a->kchain == 4) ok = apus_pre_lds_mode() == 2 && a->K == 2048 && apus_launch_pre_lds<4, true>(p, n_ent, st);
                else ok = a->K == 4096 ? apus_launch_pre_lds<8, false>(p, n_ent, st)
                                       : apus_launch_pre_lds<4, false>(p, n_ent, st);
                if (ok) return hipGetLastError();
            }
            if (a->kchain == 4) {
                if (a->K == 4096) {
                    hipLaunchKernelGGL((apus_gemm_prefill_kernel<APUS_W_FP4, 8, TT4, APUS_PRE_PD4, true>), gp, bp, 0, st, p);
                } else if (!(ra && apus_launch_pre_ra<4, true>(p, n_ent, st))) {
                    hipLaunchKernelGGL((apus_gemm_prefill_kernel<APUS_W_FP4, 4, TT4, APUS_PRE_PD4, true>), gp, bp, 0, st, p);
                }
            } else if (ra && apus_pre_ra_w13()) {
                if (a->K == 4096) { if (!apus_launch_pre_ra<8, false>(p, n_ent, st)) return hipErrorInvalidValue; }
                else              { if (!apus_launch_pre_ra<4, false>(p, n_ent, st)) return hipErrorInvalidValue; }
            } else {
                if (a->K == 4096) hipLaunchKernelGGL((apus_gemm_prefill_kernel<APUS_W_FP4, 8, TT4, APUS_PRE_PD4, false>), gp, bp, 0, st, p);
                else              hipLaunchKernelGGL((apus_gemm_prefill_kernel<APUS_W_FP4, 4, TT4, APUS_PRE_PD4, false>), gp, bp, 0, st, p);
            }
        } else {
            if (a->kchain == 4) return hipErrorInvalidValue;
            if (a->K == 4096) hipLaunchKernelGGL((apus_gemm_prefill_kernel<APUS_W_FP8, 8, 2, 2, false>), gp, bp, 0, st, p);
            else              hipLaunchKernelGGL((apus_gemm_prefill_kernel<APUS_W_FP8, 4, 2, 2, false>), gp, bp, 0, st, p);
        }
        return hipGetLastError();
    }
    /* a required accumulation order is kept by the decode and prefill
     * schedules only */
    if (a->kchain) return hipErrorInvalidValue;
    /* dense GEMMs with more than 8 rows: the tile schedule */
    if (!grouped && a->ent0.M > R && apus_fast_k(a->K) && a->O % 128 == 0) {
        /* waves per workgroup: 8 for K <= 2048, 4 above (measured best) */
#define APUS_TILE_NW(NQ) ((NQ) <= 16 ? 8 : 4)
        dim3 gt(a->O / 128, (a->ent0.M + 63) / 64, 1), bt(64 * APUS_TILE_NW(a->K / 128));
#ifndef APUS_TILE_TM
#define APUS_TILE_TM 4
#endif
#ifndef APUS_TILE_DA
#define APUS_TILE_DA 6
#endif
#ifndef APUS_TILE_PDX
#define APUS_TILE_PDX 1
#endif

#define APUS_TILE(NQ, PD) hipLaunchKernelGGL((apus_gemm_tile_kernel<WFC, NQ, (PD * APUS_TILE_PDX < NQ ? PD * APUS_TILE_PDX : NQ), APUS_TILE_DA, APUS_TILE_TM, APUS_TILE_NW(NQ)>), gt, bt, 0, st, *a)
        /* FP8 on tiled weights, plain row ranges, up to 64 rows: the narrow
         * schedule */
        if (wfmt == APUS_W_FP8 && a->wtiled && !a->ent0.arows && !a->ent0.orows && a->ent0.M <= 64 &&
            apus_narrow_on()) {
            bool ok = false;
            switch (a->K) {
            case 1024: ok = apus_launch_narrow<8>(*a, st); break;
            case 2048: ok = apus_launch_narrow<16>(*a, st); break;
            case 4096: ok = apus_launch_narrow<32>(*a, st); break;
            default:   ok = apus_launch_narrow<64>(*a, st); break;
            }
            if (ok) return hipGetLastError();
        }
        /* FP8 on tiled weights, plain row ranges: the LDS tile schedule */
        if (wfmt == APUS_W_FP8 && a->wtiled && !a->ent0.arows && !a->ent0.orows && apus_lds_tile_on()) {
            bool ok = false;
            switch (a->K) {
            case 1024: ok = apus_launch_lds_tile<8>(*a, st); break;
            case 2048: ok = apus_launch_lds_tile<16>(*a, st); break;
            case 4096: ok = apus_launch_lds_tile<32>(*a, st); break;
            default:   ok = apus_launch_lds_tile<64>(*a, st); break;
            }
            if (ok) return hipGetLastError();
        }
        if (wfmt == APUS_W_FP4) {
            constexpr int WFC = APUS_W_FP4;
            switch (a->K) {
            case 1024: APUS_TILE(8, 8); break;
            case 2048: APUS_TILE(16, 8); break;
            case 4096: APUS_TILE(32, 8); break;
            default:   APUS_TILE(64, 8); break;
            }
        } else {
            constexpr int WFC = APUS_W_FP8;
            switch (a->K) {
            case 1024: APUS_TILE(8, 6); break;
            case 2048: APUS_TILE(16, 6); break;
            case 4096: APUS_TILE(32, 6); break;
            default:   APUS_TILE(64, 6); break;
            }
        }
#undef APUS_TILE
        return hipGetLastError();
    }
    /* other grouped shapes with many row tiles */
    if (grouped && row_tiles >= 2048) {
        dim3 grid((a->O + 63) / 64, n_ent), block(256);
        const bool wide = a->max_m == 0 || a->max_m > 16;
        if (wfmt == APUS_W_FP4) {
            if (wide) hipLaunchKernelGGL((apus_gemm_stream_kernel<APUS_W_FP4, 4>), grid, block, 0, st, *a);
            else      hipLaunchKernelGGL((apus_gemm_stream_kernel<APUS_W_FP4, 1>), grid, block, 0, st, *a);
        } else {
            if (wide) hipLaunchKernelGGL((apus_gemm_stream_kernel<APUS_W_FP8, 4>), grid, block, 0, st, *a);
            else      hipLaunchKernelGGL((apus_gemm_stream_kernel<APUS_W_FP8, 1>), grid, block, 0, st, *a);
        }
        return hipGetLastError();
    }
    /* few row tiles: split K over the waves of a workgroup */
    const int nslice = (a->K / 128 + 3) / 4;
    const int nw = nslice < 8 ? nslice : 8;
    dim3 grid((a->O + 15) / 16, n_ent), block(64 * nw);
    if (wfmt == APUS_W_FP4) {
        if (grouped) hipLaunchKernelGGL((apus_gemm_kernel<APUS_W_FP4, true>), grid, block, 0, st, *a);
        else         hipLaunchKernelGGL((apus_gemm_kernel<APUS_W_FP4, false>), grid, block, 0, st, *a);
    } else {
        if (grouped) hipLaunchKernelGGL((apus_gemm_kernel<APUS_W_FP8, true>), grid, block, 0, st, *a);
        else         hipLaunchKernelGGL((apus_gemm_kernel<APUS_W_FP8, false>), grid, block, 0, st, *a);
    }
    return hipGetLastError();
}
