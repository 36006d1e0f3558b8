/*
 * apus_kernels.hip — gfx950 kernels of the HIP backend.
 *
 *  - act quant: BF16 round + per-128 E4M3 quantisation, 32 lanes (or one
 *    wave where x is not 16-byte aligned) per 128-element group
 *    (c/attn.h:393-403, c/fp4.h:293-321), bit-exact.
 *  (the block-scaled GEMMs live in apus_gemm.hip)
 *  - SwiGLU + act quant of h (c/moe.h:113-126 followed by the act quant of
 *    the w2 input, c/moe.h:309-314), 32 lanes per 128 group.
 *  - routed-pair counting sort and GEMM entry tables (c/moe.h:465-474).
 *  - (t, j)-ordered weighted accumulation (c/moe.h:148-158).
 *  - counter-based weight fill for HBM-resident synthetic experts.
 */
#include "apus_device.h"
#include "apus_internal.h"

/* ------------------------------------------------------------ act quant */

/* One wave per (row, 128-group): two elements per lane. */
__global__ __launch_bounds__(256) void apus_act_quant_kernel(
    const float *__restrict__ x, int ldx, const int32_t *__restrict__ arows,
    int M, int K, uint8_t *__restrict__ codes, float *__restrict__ scales) {
    const int nab = K >> 7;
    const int gid = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (gid >= M * nab) return;
    const int m = gid / nab, b = gid - m * nab;
    const int src = arows ? arows[m] : m;
    const float2 v = *reinterpret_cast<const float2 *>(x + (size_t)src * ldx + b * 128 + lane * 2);
    const float v0 = apus_bf16_rne(v.x), v1 = apus_bf16_rne(v.y);
    const float amax = apus_wave_max(fmaxf(fabsf(v0), fabsf(v1)));
    const uint32_t e = apus_act_scale_exp(amax);
    const float inv = apus_inv_pow2_from_exp(e);
    *reinterpret_cast<uint16_t *>(codes + (size_t)m * K + b * 128 + lane * 2) =
        (uint16_t)apus_e4m3_pack2_hw(v0 * inv, v1 * inv);
    if (lane == 0) scales[(size_t)m * nab + b] = apus_pow2_from_exp(e);
}

/* The same, 32 lanes per group, 4 elements per lane (x rows 16-byte aligned). */
__global__ __launch_bounds__(256) void apus_act_quant4_kernel(
    const float *__restrict__ x, int ldx, const int32_t *__restrict__ arows,
    int M, int K, uint8_t *__restrict__ codes, float *__restrict__ scales) {
    const int nab = K >> 7;
    const int gid = blockIdx.x * 8 + (threadIdx.x >> 5);
    const int l32 = threadIdx.x & 31;
    /* both halves of a wave take part in the shuffles: a group past the end
     * computes on a clamped group and stores nothing */
    const bool live = gid < M * nab;
    const int gq = live ? gid : M * nab - 1;
    const int m = gq / nab, b = gq - m * nab;
    const int src = arows ? arows[m] : m;
    const float4 v = *reinterpret_cast<const float4 *>(x + (size_t)src * ldx + b * 128 + l32 * 4);
    const float h[4] = {apus_bf16_rne(v.x), apus_bf16_rne(v.y), apus_bf16_rne(v.z),
                        apus_bf16_rne(v.w)};
    float amax = fmaxf(fmaxf(fabsf(h[0]), fabsf(h[1])), fmaxf(fabsf(h[2]), fabsf(h[3])));
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    const uint32_t e = apus_act_scale_exp(amax);
    const float inv = apus_inv_pow2_from_exp(e);
    if (!live) return;
    *reinterpret_cast<uint32_t *>(codes + (size_t)m * K + b * 128 + l32 * 4) =
        apus_e4m3_pack4_hw(h[0] * inv, h[1] * inv, h[2] * inv, h[3] * inv);
    if (l32 == 0) scales[(size_t)m * nab + b] = apus_pow2_from_exp(e);
}

hipError_t apus_launch_act_quant(const float *x, int ldx, const int32_t *arows,
                                 int M, int K, uint8_t *codes, float *scales,
                                 hipStream_t st) {
    if (M <= 0) return hipSuccess;
    const int groups = M * (K >> 7);
    if ((reinterpret_cast<uintptr_t>(x) & 15) == 0 && ldx % 4 == 0 &&
        (reinterpret_cast<uintptr_t>(codes) & 3) == 0) {
        hipLaunchKernelGGL(apus_act_quant4_kernel, dim3((groups + 7) / 8), dim3(256), 0, st,
                           x, ldx, arows, M, K, codes, scales);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(apus_act_quant_kernel, dim3((groups + 3) / 4), dim3(256), 0, st,
                       x, ldx, arows, M, K, codes, scales);
    return hipGetLastError();
}

/* ---------------------------------------------------- SwiGLU + act quant */

/* One 128-column group per 32 lanes (two per wave), 4 columns per lane:
 * 16-byte loads of g and u, one 4-byte store of codes. */
__global__ __launch_bounds__(256) void apus_swiglu_quant_kernel(
    const float *__restrict__ gm, const float *__restrict__ um, int M, int N,
    float limit, uint8_t *__restrict__ codes, float *__restrict__ scales) {
    const int nab = N >> 7;
    const int gid = blockIdx.x * 8 + (threadIdx.x >> 5);
    const int l32 = threadIdx.x & 31;
    /* both halves of a wave take part in the shuffles: a group past the end
     * computes on a clamped group and stores nothing */
    const bool live = gid < M * nab;
    const int gq = live ? gid : M * nab - 1;
    const int m = gq / nab, b = gq - m * nab;
    const size_t off = (size_t)m * N + b * 128 + l32 * 4;
    const float4 gv = *reinterpret_cast<const float4 *>(gm + off);
    const float4 uv = *reinterpret_cast<const float4 *>(um + off);
    const float h[4] = {apus_swiglu_h(gv.x, uv.x, limit), apus_swiglu_h(gv.y, uv.y, limit),
                        apus_swiglu_h(gv.z, uv.z, limit), apus_swiglu_h(gv.w, uv.w, limit)};
    /* h is bf16-valued, so the act quant's own BF16 round is the identity */
    float amax = fmaxf(fmaxf(fabsf(h[0]), fabsf(h[1])), fmaxf(fabsf(h[2]), fabsf(h[3])));
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    const uint32_t e = apus_act_scale_exp(amax);
    const float inv = apus_inv_pow2_from_exp(e);
    if (!live) return;
    *reinterpret_cast<uint32_t *>(codes + off) =
        apus_e4m3_pack4_hw(h[0] * inv, h[1] * inv, h[2] * inv, h[3] * inv);
    if (l32 == 0) scales[(size_t)m * nab + b] = apus_pow2_from_exp(e);
}

hipError_t apus_launch_swiglu_quant(const float *g, const float *u, int M,
                                    int N, float limit, uint8_t *codes,
                                    float *scales, hipStream_t st) {
    if (M <= 0) return hipSuccess;
    if (N <= 0 || N % 128 ||
        ((reinterpret_cast<uintptr_t>(g) | reinterpret_cast<uintptr_t>(u)) & 15) ||
        (reinterpret_cast<uintptr_t>(codes) & 3))
        return hipErrorInvalidValue;
    const int groups = M * (N >> 7);
    hipLaunchKernelGGL(apus_swiglu_quant_kernel, dim3((groups + 7) / 8), dim3(256), 0, st,
                       g, u, M, N, limit, codes, scales);
    return hipGetLastError();
}

/* ------------------------------------------------------------ MoE route */

/* Exclusive prefix sums of three ints per thread over the workgroup (at most
 * 16 waves) with one set of barriers; sw is 3 x 17 ints of LDS; total
 * receives the sums of all v. */
__device__ __forceinline__ int3 apus_block_scan3_excl(int3 v, int *sw, int3 &total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nw = (blockDim.x + 63) >> 6;
    int3 x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int a = __shfl_up(x.x, d, 64), b = __shfl_up(x.y, d, 64), c = __shfl_up(x.z, d, 64);
        if (lane >= d) { x.x += a; x.y += b; x.z += c; }
    }
    if (lane == 63) { sw[wave] = x.x; sw[17 + wave] = x.y; sw[34 + wave] = x.z; }
    __syncthreads();
    if (threadIdx.x < 3) {
        int *q = sw + 17 * threadIdx.x;
        int run = 0;
        for (int w = 0; w < nw; ++w) { const int t = q[w]; q[w] = run; run += t; }
        q[16] = run;
    }
    __syncthreads();
    const int3 r = {x.x - v.x + sw[wave], x.y - v.y + sw[17 + wave], x.z - v.z + sw[34 + wave]};
    total = int3{sw[16], sw[33], sw[50]};
    return r;
}

/* Single workgroup, one thread per expert (E <= 1024): histogram of expert
 * ids, exclusive scans, placement, entry tables. A pair among the first
 * APUS_ROUTE_REG per thread keeps its id in a register and its place inside
 * its expert is the value its histogram atomic returned (the ids are read
 * once); pairs past that window (nj > APUS_ROUTE_REG x 1024) are counted
 * after them and placed by a second atomic. Experts with 1..small_max pairs
 * are listed (in expert order) at the front of the small tables, the others
 * with pairs at the front of the large tables; the remaining slots get M = 0.
 * The order inside an expert is whatever the LDS atomics give: each output
 * row of the grouped GEMMs depends only on its own activation row, and
 * results are written back by pair id, so the order is not observable in
 * the results. */
#define APUS_ROUTE_REG 4
__global__ __launch_bounds__(1024) void apus_moe_route_kernel(
    const int32_t *__restrict__ idx, int nj, int topk, int E,
    ApusExpertTable tab, float *g, float *u, float *eo,
    int32_t *pair_sorted, int32_t *tok_sorted, ApusGemmEnt *e13s, ApusGemmEnt *e2s,
    ApusGemmEnt *e13l, ApusGemmEnt *e2l, int small_max, int2 *items13, int2 *items2,
    int n_items) {
    __shared__ int cnt[1024], base[1024], cur[1024], sw[51];
    const int e = threadIdx.x, nt = blockDim.x;
    const bool more = nj > APUS_ROUTE_REG * nt;
    /* this thread's ids and its expert's weight pointers, all in flight together */
    int qid[APUS_ROUTE_REG];
#pragma unroll
    for (int r = 0; r < APUS_ROUTE_REG; ++r) {
        const int q = e + r * nt;
        qid[r] = q < nj ? idx[q] : -1;
    }
    const int ee = e < E ? e : 0;
    const uint8_t *pw1 = tab.w1[ee], *pw1s = tab.w1s[ee], *pw3 = tab.w3[ee], *pw3s = tab.w3s[ee],
                  *pw2 = tab.w2[ee], *pw2s = tab.w2s[ee];
    cnt[e] = 0;
    __syncthreads();
    int qrank[APUS_ROUTE_REG];
#pragma unroll
    for (int r = 0; r < APUS_ROUTE_REG; ++r)
        qrank[r] = (unsigned)qid[r] < (unsigned)E ? atomicAdd(&cnt[qid[r]], 1) : 0;
    if (more) {
        __syncthreads();
        cur[e] = cnt[e];                                 /* pairs of e in the window */
        __syncthreads();
        for (int q = e + APUS_ROUTE_REG * nt; q < nj; q += nt) {
            const int id = idx[q];
            if ((unsigned)id < (unsigned)E) atomicAdd(&cnt[id], 1);
        }
    }
    __syncthreads();
    const int c = e < E ? cnt[e] : 0;
    const int small = c > 0 && c <= small_max, large = c > small_max;
    /* work list of the many-row entries: one item per APUS_PREFILL_ROWS rows */
    const int nchunk = large ? (c + APUS_PREFILL_ROWS - 1) / APUS_PREFILL_ROWS : 0;
    int3 tot;
    const int3 sc = apus_block_scan3_excl(int3{c, small | (large << 16), nchunk}, sw, tot);
    const int o0 = sc.x, packed = sc.y, cbase = sc.z;
    const int ns = tot.y & 0xffff, nl = tot.y >> 16, total_chunks = tot.z;
    base[e] = o0;
    if (more) cur[e] += o0;
    __syncthreads();
#pragma unroll
    for (int r = 0; r < APUS_ROUTE_REG; ++r) {
        if ((unsigned)qid[r] >= (unsigned)E) continue;  /* ids outside [0, E) are dropped */
        const int q = e + r * nt, pos = base[qid[r]] + qrank[r];
        pair_sorted[pos] = q;
        tok_sorted[pos] = q / topk;
    }
    if (more) {
        for (int q = e + APUS_ROUTE_REG * nt; q < nj; q += nt) {
            const int id = idx[q];
            if ((unsigned)id >= (unsigned)E) continue;
            const int pos = atomicAdd(&cur[id], 1);
            pair_sorted[pos] = q;
            tok_sorted[pos] = q / topk;
        }
    }
    if (items2) {
        for (int i = total_chunks + threadIdx.x; i < n_items; i += blockDim.x) {
            items2[i] = int2{-1, 0};
            items13[2 * i] = int2{-1, 0};
            items13[2 * i + 1] = int2{-1, 0};
        }
    }
    if (e >= E) return;
    ApusGemmEnt a;
    a.arows = tok_sorted + o0; a.orows = nullptr; a.a0 = 0; a.o0 = o0; a.M = c; a.pad = 0;
    ApusGemmEnt b;
    b.w = pw2; b.ws = pw2s; b.out = eo;
    b.arows = nullptr; b.orows = pair_sorted + o0; b.a0 = o0; b.o0 = 0; b.M = c; b.pad = 0;
    if (small | large) {
        const int slot = small ? (packed & 0xffff) : (packed >> 16);
        ApusGemmEnt *t13 = small ? e13s : e13l;
        a.w = pw1; a.ws = pw1s; a.out = g;
        t13[2 * slot] = a;
        a.w = pw3; a.ws = pw3s; a.out = u;
        t13[2 * slot + 1] = a;
        (small ? e2s : e2l)[slot] = b;
    }
    ApusGemmEnt z{};
    if (e >= ns) { e13s[2 * e] = z; e13s[2 * e + 1] = z; e2s[e] = z; }
    if (e >= nl) { e13l[2 * e] = z; e13l[2 * e + 1] = z; e2l[e] = z; }
    if (items2) {
        const int slot = packed >> 16;
        for (int k = 0; k < nchunk && cbase + k < n_items; ++k) {
            const int c0 = k * APUS_PREFILL_ROWS;
            items2[cbase + k] = int2{slot, c0};
            items13[2 * (cbase + k)] = int2{2 * slot, c0};
            items13[2 * (cbase + k) + 1] = int2{2 * slot + 1, c0};
        }
    }
}

hipError_t apus_launch_moe_route(const int32_t *idx, int nj, int topk, int E,
                                 ApusExpertTable tab, float *g, float *u, float *eo,
                                 int32_t *pair_sorted, int32_t *tok_sorted,
                                 ApusGemmEnt *e13s, ApusGemmEnt *e2s, ApusGemmEnt *e13l,
                                 ApusGemmEnt *e2l, int small_max, int2 *items13, int2 *items2,
                                 int n_items, hipStream_t st) {
    if (E <= 0 || E > 1024) return hipErrorInvalidValue;
    hipLaunchKernelGGL(apus_moe_route_kernel, dim3(1), dim3(1024), 0, st, idx, nj, topk, E,
                       tab, g, u, eo, pair_sorted, tok_sorted, e13s, e2s, e13l, e2l, small_max,
                       items13, items2, n_items);
    return hipGetLastError();
}

/* ---------------------------------------------------------------- router */

/* Router scores (c/moe.h:352-367): sp[t, e] = sqrt(softplus(gate_w[e] . x[t]))
 * and, with a bias, biased = sp + bias[e] for the selection. One workgroup
 * per (expert, group of up to 8 tokens): the expert's gate row is read once
 * into registers (thread i holds float4s i, i + 256, ...), each token's dot is
 * a per-thread partial, a fixed xor-shuffle tree per wave and the four wave
 * sums in wave order. The fp32 sum order differs from the reference's
 * sequential dot (and expf/log1pf come from ROCm's libm), so scores match
 * within fp32 rounding, not bitwise. dim % 256 == 0, dim <= 8192. */
#define APUS_ROUTER_TT 8
__global__ __launch_bounds__(256) void apus_router_kernel(
    const float *__restrict__ gate_w, const float *__restrict__ bias,
    const float *__restrict__ x, int s, int dim, int E, float *__restrict__ sp,
    float *__restrict__ biased) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int e = blockIdx.x, t0 = blockIdx.y * APUS_ROUTER_TT;
    const int nt = min(APUS_ROUTER_TT, s - t0);
    const int n4 = dim >> 2;
    const float4 *wr = reinterpret_cast<const float4 *>(gate_w + (size_t)e * dim);
    float4 g[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
        g[i] = (tid + 256 * i < n4) ? apus_gld<float4>(wr + tid + 256 * i)
                                    : make_float4(0.f, 0.f, 0.f, 0.f);
    float acc[APUS_ROUTER_TT];
#pragma unroll
    for (int t = 0; t < APUS_ROUTER_TT; ++t) {
        acc[t] = 0.0f;
        if (t < nt) {
            const float4 *xr = reinterpret_cast<const float4 *>(x + (size_t)(t0 + t) * dim);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (tid + 256 * i < n4) {
                    const float4 a = apus_gld<float4>(xr + tid + 256 * i);
                    acc[t] = acc[t] + a.x * g[i].x;
                    acc[t] = acc[t] + a.y * g[i].y;
                    acc[t] = acc[t] + a.z * g[i].z;
                    acc[t] = acc[t] + a.w * g[i].w;
                }
            }
        }
    }
    __shared__ float part[4][APUS_ROUTER_TT];
#pragma unroll
    for (int t = 0; t < APUS_ROUTER_TT; ++t) {
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) acc[t] = acc[t] + __shfl_xor(acc[t], off, 64);
        if (lane == 0) part[wv][t] = acc[t];
    }
    __syncthreads();
    if (tid < nt) {
        const float d = ((part[0][tid] + part[1][tid]) + part[2][tid]) + part[3][tid];
        const float v = d > 20.0f ? d : log1pf(expf(d));
        const float r = sqrtf(v);
        const size_t o = (size_t)(t0 + tid) * E + e;
        sp[o] = r;
        if (biased) biased[o] = r + bias[e];
    }
}

/* The same scores for more than 8 tokens: one workgroup per (8 experts, 8
 * tokens), so each gate row and each x row is read by s/8 and E/8 workgroups
 * instead of every x row by all E. Thread i takes the same K elements in the
 * same order as above (float4s i, i + 256, ...) for its 64 (expert, token)
 * dots; the xor-shuffle tree is computed as a reduce-scatter (at each step a
 * lane adds its partner's half of the values it keeps, so after six steps
 * lane l holds dot l, every addition the one the tree makes), then the four
 * wave sums in wave order: every score equals the one-expert kernel's bit for
 * bit. dim % 1024 == 0, dim <= 8192, E % 8 == 0. */
__global__ __launch_bounds__(256) void apus_router8_kernel(
    const float *__restrict__ gate_w, const float *__restrict__ bias,
    const float *__restrict__ x, int s, int dim, int E, float *__restrict__ sp,
    float *__restrict__ biased) {
    constexpr int EG = 8, TT = APUS_ROUTER_TT;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int e0 = blockIdx.x * EG, t0 = blockIdx.y * TT;
    float v[EG * TT];                                     /* index i * TT + t */
#pragma unroll
    for (int q = 0; q < EG * TT; ++q) v[q] = 0.0f;
    for (int k = tid * 4; k < dim; k += 1024) {
        float4 g[EG], a[TT];
#pragma unroll
        for (int i = 0; i < EG; ++i) g[i] = apus_gld<float4>(gate_w + (size_t)(e0 + i) * dim + k);
#pragma unroll
        for (int t = 0; t < TT; ++t)
            a[t] = apus_gld<float4>(x + (size_t)min(t0 + t, s - 1) * dim + k);
#pragma unroll
        for (int i = 0; i < EG; ++i)
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                float &c = v[i * TT + t];
                c = c + a[t].x * g[i].x;
                c = c + a[t].y * g[i].y;
                c = c + a[t].z * g[i].z;
                c = c + a[t].w * g[i].w;
            }
    }
    /* reduce-scatter over the wave: step `off` keeps the upper half of the
     * remaining values in lanes with that bit set, the lower half elsewhere */
#pragma unroll
    for (int off = 32, n = 64; off >= 1; off >>= 1, n >>= 1) {
        const bool up = lane & off;
#pragma unroll
        for (int j = 0; j < n / 2; ++j) {
            const float send = up ? v[j] : v[j + n / 2];
            const float keep = up ? v[j + n / 2] : v[j];
            v[j] = keep + __shfl_xor(send, off, 64);
        }
    }
    __shared__ float part[4][EG * TT];
    part[wv][lane] = v[0];                                /* dot `lane` */
    __syncthreads();
    if (tid < EG * TT) {
        const int i = tid / TT, t = tid % TT;
        if (t0 + t < s) {
            const float d = ((part[0][tid] + part[1][tid]) + part[2][tid]) + part[3][tid];
            const float u = d > 20.0f ? d : log1pf(expf(d));
            const float r = sqrtf(u);
            const size_t o = (size_t)(t0 + t) * E + e0 + i;
            sp[o] = r;
            if (biased) biased[o] = r + bias[e0 + i];
        }
    }
}

hipError_t apus_launch_router(const float *gate_w, const float *bias, const float *x, int s,
                              int dim, int E, float *sp, float *biased, hipStream_t st) {
    if (s <= 0) return hipSuccess;
    if (dim % 256 || dim > 8192 || E <= 0) return hipErrorInvalidValue;
    if (s > APUS_ROUTER_TT && dim % 1024 == 0 && E % 8 == 0) {
        hipLaunchKernelGGL(apus_router8_kernel, dim3(E / 8, (s + APUS_ROUTER_TT - 1) / APUS_ROUTER_TT),
                           dim3(256), 0, st, gate_w, bias, x, s, dim, E, sp, biased);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(apus_router_kernel, dim3(E, (s + APUS_ROUTER_TT - 1) / APUS_ROUTER_TT),
                       dim3(256), 0, st, gate_w, bias, x, s, dim, E, sp, biased);
    return hipGetLastError();
}

/* Expert choice and weights of one token per workgroup (apus_route_token;
 * c/moe.h:384-410): idx[t, j] and wgt[t, j] = sp[idx[t, j]] / sum * route_scale. */
__global__ __launch_bounds__(256) void apus_topk_kernel(
    const float *__restrict__ sel, const float *__restrict__ sp, int E, int topk,
    const int64_t *__restrict__ tid2eid, const int64_t *__restrict__ ids, float route_scale,
    int32_t *__restrict__ idx, float *__restrict__ wgt) {
    const int t = blockIdx.x, tid = threadIdx.x;
    __shared__ __align__(16) uint64_t lk[1024];
    __shared__ int32_t chosen[16];
    __shared__ float chp[16];
    apus_route_token(tid2eid ? nullptr : sel + (size_t)t * E, sp + (size_t)t * E, E, topk,
                     tid2eid ? tid2eid + ids[t] * topk : nullptr, lk, chosen, chp);
    if (tid < topk) {
        idx[t * topk + tid] = chosen[tid];
        wgt[t * topk + tid] = apus_route_weight(chp, topk, tid, route_scale);
    }
}

hipError_t apus_launch_topk(const float *sel, const float *sp, int s, int E, int topk,
                            const int64_t *tid2eid, const int64_t *ids, float route_scale,
                            int32_t *idx, float *wgt, hipStream_t st) {
    if (s <= 0) return hipSuccess;
    if (E <= 0 || E > 1024 || topk <= 0 || topk > 16 || topk > E) return hipErrorInvalidValue;
    hipLaunchKernelGGL(apus_topk_kernel, dim3(s), dim3(256), 0, st, sel, sp, E, topk, tid2eid, ids,
                       route_scale, idx, wgt);
    return hipGetLastError();
}

/* out = bf16(a + b), elementwise (c/moe.h:588-589) */
__global__ __launch_bounds__(256) void apus_add_bf16_kernel(const float *__restrict__ a,
                                                            const float *__restrict__ b,
                                                            float *__restrict__ out, size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = apus_bf16_rne(a[i] + b[i]);
}

hipError_t apus_launch_add_bf16(const float *a, const float *b, float *out, size_t n,
                                hipStream_t st) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(apus_add_bf16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       a, b, out, n);
    return hipGetLastError();
}

/* ------------------------------------------------------- MoE accumulate */

__global__ __launch_bounds__(256) void apus_moe_accum_kernel(
    const float *__restrict__ eo, const float *__restrict__ wgt, int s,
    int topk, int dim, float *__restrict__ y, const float *__restrict__ add_src,
    float *__restrict__ add_out) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int t = blockIdx.y;
    if (i >= dim) return;
    float acc = 0.0f;
    for (int j = 0; j < topk; ++j) {
        const float p = __fmul_rn(wgt[t * topk + j], eo[(size_t)(t * topk + j) * dim + i]);
        acc = __fadd_rn(acc, p);
    }
    y[(size_t)t * dim + i] = acc;
    /* optional: the sublayer output bf16(y + shared) (c/moe.h:588-589) */
    if (add_out) add_out[(size_t)t * dim + i] = apus_bf16_rne(acc + add_src[(size_t)t * dim + i]);
    (void)s;
}

/* The same sums, 4 columns per thread (16-byte loads and stores; dim % 4 == 0). */
__global__ __launch_bounds__(256) void apus_moe_accum4_kernel(
    const float *__restrict__ eo, const float *__restrict__ wgt, int topk, int dim,
    float *__restrict__ y, const float *__restrict__ add_src, float *__restrict__ add_out) {
    const int i = (blockIdx.x * 256 + threadIdx.x) * 4;
    const int t = blockIdx.y;
    if (i >= dim) return;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int j = 0; j < topk; ++j) {
        const float w = wgt[t * topk + j];
        const float4 v = *reinterpret_cast<const float4 *>(eo + (size_t)(t * topk + j) * dim + i);
        acc[0] = __fadd_rn(acc[0], __fmul_rn(w, v.x));
        acc[1] = __fadd_rn(acc[1], __fmul_rn(w, v.y));
        acc[2] = __fadd_rn(acc[2], __fmul_rn(w, v.z));
        acc[3] = __fadd_rn(acc[3], __fmul_rn(w, v.w));
    }
    const size_t o = (size_t)t * dim + i;
    *reinterpret_cast<float4 *>(y + o) = float4{acc[0], acc[1], acc[2], acc[3]};
    if (add_out) {
        const float4 a = *reinterpret_cast<const float4 *>(add_src + o);
        *reinterpret_cast<float4 *>(add_out + o) =
            float4{apus_bf16_rne(acc[0] + a.x), apus_bf16_rne(acc[1] + a.y),
                   apus_bf16_rne(acc[2] + a.z), apus_bf16_rne(acc[3] + a.w)};
    }
}

hipError_t apus_launch_moe_accum(const float *eo, const float *wgt, int s,
                                 int topk, int dim, float *y, const float *add_src,
                                 float *add_out, hipStream_t st) {
    if (s <= 0) return hipSuccess;
    const bool al = ((reinterpret_cast<uintptr_t>(eo) | reinterpret_cast<uintptr_t>(y) |
                      reinterpret_cast<uintptr_t>(add_src) | reinterpret_cast<uintptr_t>(add_out)) &
                     15) == 0;
    if (dim % 4 == 0 && al) {
        hipLaunchKernelGGL(apus_moe_accum4_kernel, dim3((dim / 4 + 255) / 256, s), dim3(256), 0, st,
                           eo, wgt, topk, dim, y, add_src, add_out);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(apus_moe_accum_kernel, dim3((dim + 255) / 256, s), dim3(256), 0, st,
                       eo, wgt, s, topk, dim, y, add_src, add_out);
    return hipGetLastError();
}

/* ------------------------------------------------- plain-weight GEMV */

/* Plain-weight linears (c/attn.h:600-666 apus_f32_linear / apus_bf16_linear,
 * the wo_a rows of the f32_linear hook, c/model.h:585-647 apus_head_gemv):
 * FP32 or BF16 weights, FP32 accumulation. A wave owns 4 output rows and
 * sweeps K in 512-element steps, each lane taking 8 consecutive elements
 * per row (one 16-byte BF16 load or two FP32 loads), against up to 8 rows
 * of x (one row in the M = 1 instance); lane partials meet in a fixed xor-shuffle tree. The CPU sums each
 * row sequentially, so results agree within FP32 summation error, not
 * bitwise. Launch row y covers x rows [MB y, MB y + MB). */
#ifndef APUS_WG_NR
#define APUS_WG_NR 4
#endif
template <bool WB, int MB>
__global__ __launch_bounds__(256) void apus_wgemv_kernel(const void *__restrict__ w,
                                                         const float *__restrict__ x,
                                                         float *__restrict__ out, int M, int K,
                                                         int O, int flags) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int o0 = (blockIdx.x * 4 + wave) * APUS_WG_NR;
    const int m0 = blockIdx.y * MB;
    const int mb = min(MB, M - m0);
    const bool rin = flags & 1;
    float acc[MB][APUS_WG_NR];
#pragma unroll
    for (int m = 0; m < MB; ++m)
#pragma unroll
        for (int r = 0; r < APUS_WG_NR; ++r) acc[m][r] = 0.0f;
    for (int k = lane * 8; k < K; k += 512) {
        float wv[APUS_WG_NR][8];
#pragma unroll
        for (int r = 0; r < APUS_WG_NR; ++r) {
            const int o = min(o0 + r, O - 1);
            if constexpr (WB) {
                const uint4 u = apus_gld<uint4>((const uint16_t *)w + (size_t)o * K + k);
                const unsigned q[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    wv[r][2 * i] = __uint_as_float(q[i] << 16);
                    wv[r][2 * i + 1] = __uint_as_float(q[i] & 0xffff0000u);
                }
            } else {
                const float *p = (const float *)w + (size_t)o * K + k;
                const float4 a = apus_gld<float4>(p), b = apus_gld<float4>(p + 4);
                wv[r][0] = a.x; wv[r][1] = a.y; wv[r][2] = a.z; wv[r][3] = a.w;
                wv[r][4] = b.x; wv[r][5] = b.y; wv[r][6] = b.z; wv[r][7] = b.w;
            }
        }
#pragma unroll
        for (int m = 0; m < MB; ++m) {
            if (m < mb) {
                const float *p = x + (size_t)(m0 + m) * K + k;
                const float4 a = apus_gld<float4>(p), b = apus_gld<float4>(p + 4);
                float xv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
                if (rin) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) xv[i] = apus_bf16_rne(xv[i]);
                }
#pragma unroll
                for (int r = 0; r < APUS_WG_NR; ++r)
#pragma unroll
                    for (int i = 0; i < 8; ++i) acc[m][r] = __builtin_fmaf(wv[r][i], xv[i], acc[m][r]);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MB; ++m) {
        if (m < mb) {
#pragma unroll
            for (int r = 0; r < APUS_WG_NR; ++r) {
                float v = acc[m][r];
#pragma unroll
                for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
                if (lane == 0 && o0 + r < O)
                    out[(size_t)(m0 + m) * O + o0 + r] = (flags & 2) ? apus_bf16_rne(v) : v;
            }
        }
    }
}

/* One x row against BF16 weights with K = 512 NS (the LM head at dim 4096;
 * c/model.h:585-647 apus_head_gemv, c/attn.h:600-666 apus_bf16_linear):
 * x is staged once per workgroup in LDS (fp32, BF16-rounded first with flag
 * 1), so each wave reads it from there for its NR rows instead of from L2
 * (the general kernel reads the 16 KB row once per 4 weight rows: half as
 * many bytes again as the weights, through L2). Lane l takes elements
 * 8 l .. 8 l + 7 of each 512-step (one 16-byte load per row, streamed, a
 * ring PD steps deep); x sits in LDS as [step][half][lane][4] so its two
 * 16-byte reads per step are contiguous over the lanes. Lane partials meet
 * in a fixed xor-shuffle tree, as in apus_wgemv_kernel (within FP32
 * summation error of the CPU's sequential sums, not bitwise). */
template <int NS, int NR, int PD>
__global__ __launch_bounds__(256) void apus_head_kernel(const uint16_t *__restrict__ w,
                                                        const float *__restrict__ x,
                                                        float *__restrict__ out, int O, int flags) {
    constexpr int K = NS * 512;
    __shared__ __align__(16) float hx[K];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int o0 = (blockIdx.x * 4 + wave) * NR;
    /* x first (L2 hits), then the weight ring */
    float4 xv[K / 1024];
#pragma unroll
    for (int j = 0; j < K / 1024; ++j) xv[j] = apus_gld<float4>(x + (size_t)(threadIdx.x + 256 * j) * 4);
    /* 32-bit byte offsets from the (uniform) weight base: one VGPR a row
     * (O K 2 < 4 GiB is checked by the launcher) */
    const uint8_t *wb = reinterpret_cast<const uint8_t *>(w);
    unsigned wo[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) wo[r] = (unsigned)min(o0 + r, O - 1) * (unsigned)(K * 2) + (unsigned)lane * 16u;
    apus_v4u ring[PD][NR];
#pragma unroll
    for (int u = 0; u < PD; ++u)
#pragma unroll
        for (int r = 0; r < NR; ++r) ring[u][r] = apus_ld16_stream(wb + (wo[r] + u * 1024u));
#pragma unroll
    for (int j = 0; j < K / 1024; ++j) {
        float4 v = xv[j];
        if (flags & 1) {
            v.x = apus_bf16_rne(v.x); v.y = apus_bf16_rne(v.y);
            v.z = apus_bf16_rne(v.z); v.w = apus_bf16_rne(v.w);
        }
        const int e = (threadIdx.x + 256 * j) * 4;          /* element of x */
        const int st = e >> 9, l = (e & 511) >> 3, h = (e >> 2) & 1;
        *reinterpret_cast<float4 *>(&hx[((st * 2 + h) * 64 + l) * 4]) = v;
    }
    apus_lds_barrier();
    float acc[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int st = 0; st < NS; ++st) {
        const float4 a = *reinterpret_cast<const float4 *>(&hx[((st * 2) * 64 + lane) * 4]);
        const float4 b = *reinterpret_cast<const float4 *>(&hx[((st * 2 + 1) * 64 + lane) * 4]);
        const float xe[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        apus_v4u (&cur)[NR] = ring[st % PD];
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const unsigned q[4] = {cur[r].x, cur[r].y, cur[r].z, cur[r].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                acc[r] = __builtin_fmaf(__uint_as_float(q[i] << 16), xe[2 * i], acc[r]);
                acc[r] = __builtin_fmaf(__uint_as_float(q[i] & 0xffff0000u), xe[2 * i + 1], acc[r]);
            }
        }
        /* the step's FMAs stay here (sunk to the reduction, they kept every
         * step's weights live) */
#pragma unroll
        for (int r = 0; r < NR; ++r) asm volatile("" : "+v"(acc[r]));
        if (st + PD < NS) {
#pragma unroll
            for (int r = 0; r < NR; ++r) cur[r] = apus_ld16_stream(wb + (wo[r] + (st + PD) * 1024u));
        }
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        float v = acc[r];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
        if (lane == 0 && o0 + r < O) out[o0 + r] = (flags & 2) ? apus_bf16_rne(v) : v;
    }
}

hipError_t apus_launch_wgemv(const void *w, const float *x, float *out, int M, int K, int O,
                             int flags, hipStream_t st) {
    if (M <= 0 || O <= 0) return hipSuccess;
    if (K <= 0 || K % 8) return hipErrorInvalidValue;
    /* one x row, BF16 weights, K 2048 / 4096 / 8192: x staged in LDS, 4
     * rows a wave, a ring 4 steps deep (LM head [129280, 4096]: 154-158
     * against 176 us for the general kernel; 8 rows a wave or rings of 3, 6,
     * 8 steps 157-161 us) */
    if (M == 1 && (flags & 4) && (K == 2048 || K == 4096 || K == 8192) && (size_t)O * K * 2 < (1ull << 32)) {
        constexpr int NR = 4, PD = 4;
        const dim3 grid((O + 4 * NR - 1) / (4 * NR));
        const uint16_t *wh = (const uint16_t *)w;
        if (K == 2048)      hipLaunchKernelGGL((apus_head_kernel<4, NR, PD>), grid, dim3(256), 0, st, wh, x, out, O, flags);
        else if (K == 4096) hipLaunchKernelGGL((apus_head_kernel<8, NR, PD>), grid, dim3(256), 0, st, wh, x, out, O, flags);
        else                hipLaunchKernelGGL((apus_head_kernel<16, NR, PD>), grid, dim3(256), 0, st, wh, x, out, O, flags);
        return hipGetLastError();
    }
    const unsigned gx = (O + 4 * APUS_WG_NR - 1) / (4 * APUS_WG_NR);
    const dim3 block(256);
    if (M == 1) {       /* decode (the LM head): accumulators for one x row */
        if (flags & 4) hipLaunchKernelGGL((apus_wgemv_kernel<true, 1>), dim3(gx), block, 0, st, w, x, out, M, K, O, flags);
        else           hipLaunchKernelGGL((apus_wgemv_kernel<false, 1>), dim3(gx), block, 0, st, w, x, out, M, K, O, flags);
        return hipGetLastError();
    }
    const dim3 grid(gx, (M + 7) / 8);
    if (flags & 4) hipLaunchKernelGGL((apus_wgemv_kernel<true, 8>), grid, block, 0, st, w, x, out, M, K, O, flags);
    else           hipLaunchKernelGGL((apus_wgemv_kernel<false, 8>), grid, block, 0, st, w, x, out, M, K, O, flags);
    return hipGetLastError();
}

/* ------------------------------------------------- E4M3 conversion check */

/* Every fp32 input x with |x| <= 448 (both signs): the hardware conversion
 * (apus_e4m3_pack4_hw) against apus_e4m3_code; counts mismatches and keeps
 * the largest mismatching input bits. */
__global__ __launch_bounds__(256) void apus_e4m3_hw_check_kernel(uint32_t n, unsigned *bad,
                                                                 unsigned *last_bad) {
    const uint32_t i0 = (blockIdx.x * 256u + threadIdx.x) * 2u;
    unsigned nbad = 0, lb = 0;
    if (i0 < n) {
        const float x0 = __uint_as_float(i0), x1 = __uint_as_float(i0 + 1 < n ? i0 + 1 : i0);
        const uint32_t hw = apus_e4m3_pack4_hw(x0, x1, -x0, -x1);
        const uint32_t sw = apus_e4m3_code(x0) | (apus_e4m3_code(x1) << 8) |
                            (apus_e4m3_code(-x0) << 16) | (apus_e4m3_code(-x1) << 24);
        if (hw != sw) { nbad = 1; lb = i0; }
    }
    if (nbad) {
        __hip_atomic_fetch_add(bad, nbad, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_fetch_max(last_bad, lb, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

hipError_t apus_launch_e4m3_hw_check(unsigned *bad, unsigned *last_bad, hipStream_t st) {
    const uint32_t n = 0x43e00001u;                  /* bits of 448.0f, inclusive */
    const uint32_t pairs = (n + 1) / 2;
    hipLaunchKernelGGL(apus_e4m3_hw_check_kernel, dim3((pairs + 255) / 256), dim3(256), 0, st, n,
                       bad, last_bad);
    return hipGetLastError();
}

/* ------------------------------------------------------------------ fill */

__device__ __forceinline__ uint64_t apus_hash64(uint64_t seed, uint64_t stream,
                                                uint64_t index) {
    uint64_t z = seed * 0x9e3779b97f4a7c15ull + stream * 0xd1b54a32d192ed03ull +
                 index * 0xbf58476d1ce4e5b9ull + 0x94d049bb133111ebull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

/* Each thread fills 8 consecutive bytes starting at first + 8*tid. */
__global__ __launch_bounds__(256) void apus_fill_kernel(uint8_t *dst, size_t n,
                                                        uint64_t seed, uint64_t sid,
                                                        uint64_t first, int kind) {
    const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t i0 = t * 8;
    if (i0 >= n) return;
    uint8_t b[8];
    if (kind == 0 && ((first & 7) == 0)) {
        const uint64_t h = apus_hash64(seed, sid, (first + i0) >> 3);
#pragma unroll
        for (int k = 0; k < 8; ++k) b[k] = (uint8_t)(h >> (8 * k));
    } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint64_t pos = first + i0 + k;
            if (kind == 0) { b[k] = (uint8_t)(apus_hash64(seed, sid, pos >> 3) >> (8 * (pos & 7))); continue; }
            const uint64_t h = apus_hash64(seed, sid, pos);
            if (kind == 1) b[k] = (uint8_t)(118u + (uint32_t)((h >> 32) % 13u));
            else if (kind == 2) {
                const int32_t sum = (int32_t)(h & 0xffff) + (int32_t)((h >> 16) & 0xffff) +
                                    (int32_t)((h >> 32) & 0xffff) + (int32_t)(h >> 48);
                const float v = __fmul_rn((float)(sum - 131070), 1.0f / 37837.6f);
                b[k] = (uint8_t)apus_e4m3_code(v);
            } else b[k] = (uint8_t)(117u + (uint32_t)((h >> 32) % 7u));
        }
    }
    if (i0 + 8 <= n && ((reinterpret_cast<uintptr_t>(dst + i0) & 7) == 0)) {
        uint64_t v = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) v |= (uint64_t)b[k] << (8 * k);
        *reinterpret_cast<uint64_t *>(dst + i0) = v;
    } else {
        for (int k = 0; k < 8 && i0 + k < n; ++k) dst[i0 + k] = b[k];
    }
}

hipError_t apus_launch_fill(uint8_t *dst, size_t n, uint64_t seed,
                            uint64_t stream_id, uint64_t first, int kind,
                            hipStream_t st) {
    if (!n) return hipSuccess;
    const size_t threads = (n + 7) / 8;
    const size_t max_blocks = (size_t)1 << 30;
    for (size_t done = 0; done < threads;) {
        size_t nb = (threads - done + 255) / 256;
        if (nb > max_blocks) nb = max_blocks;
        const size_t bytes0 = done * 8;
        hipLaunchKernelGGL(apus_fill_kernel, dim3((unsigned)nb), dim3(256), 0, st,
                           dst + bytes0, n - bytes0, seed, stream_id, first + bytes0, kind);
        done += nb * 256;
    }
    return hipGetLastError();
}

/* One tensor (w or its E8M0 scales) of every expert of an expert-store layer,
 * generated straight into the store's layout: expert e's tensor at
 * base + e * stride, stream id sid0 + 8 e. Each thread writes one 16-byte
 * piece: it finds the piece's row-major position (the MFMA-tiled layout of
 * apus_pack_kernel when tiled) and generates the 16 bytes the counter fill
 * would have put there, so the result equals fill-then-pack byte for byte.
 * what: 0 = MXFP4 weights [O, K/2] (kind 0), 1 = E8M0 scales [O, K/32]
 * (kind 1). */
__global__ __launch_bounds__(256) void apus_store_fill_kernel(uint8_t *base, size_t stride, int O,
                                                              int K, int what, int tiled,
                                                              uint64_t seed, uint64_t sid0) {
    const int e = blockIdx.y;
    const size_t c = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t rb = what ? (size_t)K / 32 : (size_t)K / 2, n = (size_t)O * rb;
    if (c * 16 >= n) return;
    size_t row = 0, col = c * 16;          /* row-major: position c * 16 */
    if (!tiled) {
    } else if (what == 0) {
        const int NQ = K >> 7, lane = (int)(c & 63);
        const size_t rest = c >> 6;
        row = (rest / NQ) * 16 + (lane & 15);
        col = (rest % NQ) * 64 + (lane >> 4) * 16;
    } else {
        const int NS = K >> 9;
        const size_t rest = c >> 4;
        row = (rest / NS) * 16 + (c & 15);
        col = (rest % NS) * 16;
    }
    const uint64_t sid = sid0 + (uint64_t)e * 8, pos = row * rb + col;
    uint32_t w[4];
    if (what == 0) {
        const uint64_t h0 = apus_hash64(seed, sid, pos >> 3), h1 = apus_hash64(seed, sid, (pos >> 3) + 1);
        w[0] = (uint32_t)h0; w[1] = (uint32_t)(h0 >> 32); w[2] = (uint32_t)h1; w[3] = (uint32_t)(h1 >> 32);
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t v = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint64_t h = apus_hash64(seed, sid, pos + 4 * i + k);
                v |= (118u + (uint32_t)((h >> 32) % 13u)) << (8 * k);
            }
            w[i] = v;
        }
    }
    uint8_t *dst = base + (size_t)e * stride + c * 16;
    if (c * 16 + 16 <= n) {
        *reinterpret_cast<uint4 *>(dst) = uint4{w[0], w[1], w[2], w[3]};
    } else {
        for (size_t k = 0; c * 16 + k < n; ++k) dst[k] = (uint8_t)(w[k >> 2] >> (8 * (k & 3)));
    }
}

hipError_t apus_launch_store_fill(uint8_t *base, size_t stride, int E, int O, int K, int what,
                                  int tiled, uint64_t seed, uint64_t sid0, hipStream_t st) {
    if (E <= 0 || O <= 0 || K <= 0 || K % 32 || (tiled && (O % 16 || K % 512)) || stride % 16 ||
        reinterpret_cast<uintptr_t>(base) % 16)
        return hipErrorInvalidValue;
    const size_t pieces = ((size_t)O * (what ? (size_t)K / 32 : (size_t)K / 2) + 15) / 16;
    hipLaunchKernelGGL(apus_store_fill_kernel, dim3((unsigned)((pieces + 255) / 256), (unsigned)E),
                       dim3(256), 0, st, base, stride, O, K, what, tiled, seed, sid0);
    return hipGetLastError();
}

/* ------------------------------------------------- MFMA-tiled weight layout */

/* One thread per 16-byte piece of the tiled layout: FP4 weights
 * [O/16][K/128][64 lanes][16 B], FP8 weights [O/16][K/128][2][64 lanes][16 B]
 * (lane = r + 16 g holds bytes [16 g, +16) of the group's first or second
 * 64-byte half of row 16 t + r), then FP4 scales [O/16][K/512][16 rows][16 B].
 * unpack != 0 runs the map backwards. */
__global__ __launch_bounds__(256) void apus_pack_kernel(
    const uint8_t *__restrict__ src, const uint8_t *__restrict__ ssrc, uint8_t *__restrict__ dst,
    uint8_t *__restrict__ sdst, int fp8, int O, int K, int unpack) {
    const size_t c = (size_t)blockIdx.x * 256 + threadIdx.x;
    const int NQ = K >> 7, NS = K >> 9;
    const size_t rb = fp8 ? (size_t)K : (size_t)K / 2;
    const size_t nw = (size_t)O * rb / 16;                   /* weight pieces */
    const size_t ns = fp8 ? 0 : (size_t)O * (K / 32) / 16;   /* FP4 scale pieces */
    if (c < nw) {
        const int lane = (int)(c & 63);
        size_t rest = c >> 6;
        int h = 0;
        if (fp8) { h = (int)(rest & 1); rest >>= 1; }
        const int q = (int)(rest % NQ);
        const size_t t = rest / NQ;
        const size_t o = t * 16 + (lane & 15);
        const size_t rm = o * rb + (fp8 ? (size_t)q * 128 + h * 64 : (size_t)q * 64) + (lane >> 4) * 16;
        const size_t tm = c * 16;
        if (unpack) *reinterpret_cast<uint4 *>(dst + rm) = *reinterpret_cast<const uint4 *>(src + tm);
        else        *reinterpret_cast<uint4 *>(dst + tm) = *reinterpret_cast<const uint4 *>(src + rm);
    } else if (c < nw + ns) {
        const size_t d = c - nw;
        const int r = (int)(d & 15);
        const size_t rest = d >> 4;
        const int sl = (int)(rest % NS);
        const size_t t = rest / NS;
        const size_t rm = (t * 16 + r) * (size_t)(K / 32) + sl * 16;
        const size_t tm = d * 16;
        if (unpack) *reinterpret_cast<uint4 *>(sdst + rm) = *reinterpret_cast<const uint4 *>(ssrc + tm);
        else        *reinterpret_cast<uint4 *>(sdst + tm) = *reinterpret_cast<const uint4 *>(ssrc + rm);
    }
}

hipError_t apus_launch_pack(int wfmt, const uint8_t *w, const uint8_t *ws, uint8_t *tw,
                            uint8_t *tws, int O, int K, int unpack, hipStream_t st) {
    if (O <= 0 || O % 16 || K <= 0 || K % 512) return hipErrorInvalidValue;
    const bool fp8 = wfmt == APUS_W_FP8;
    const size_t rb = fp8 ? (size_t)K : (size_t)K / 2;
    const size_t n = (size_t)O * rb / 16 + (fp8 ? 0 : (size_t)O * (K / 32) / 16);
    hipLaunchKernelGGL(apus_pack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       w, ws, tw, tws, fp8 ? 1 : 0, O, K, unpack);
    return hipGetLastError();
}

/* ------------------------------------------------------------ bf16 round */

__global__ __launch_bounds__(256) void apus_bf16_round_kernel(float *v, size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) v[i] = apus_bf16_rne(v[i]);
}

hipError_t apus_launch_bf16_round(float *v, size_t n, hipStream_t st) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(apus_bf16_round_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, v, n);
    return hipGetLastError();
}

/* ------------------------------------------------------------ delay */

/* One wave that sleeps until `ticks` of the constant-rate wall clock have
 * passed (bounded: at most 2^20 sleep rounds of ~3 us, so it ends even if
 * the clock were to stand still). Used by the timer to hold the stream
 * while the host queues the work to be timed. */
__global__ __launch_bounds__(64) void apus_delay_kernel(unsigned long long ticks) {
    const unsigned long long t0 = wall_clock64();
    for (unsigned it = 0; it < (1u << 20); ++it) {
        if (wall_clock64() - t0 >= ticks) break;
        __builtin_amdgcn_s_sleep(127);
    }
}

hipError_t apus_launch_delay(unsigned long long ticks, hipStream_t st) {
    hipLaunchKernelGGL(apus_delay_kernel, dim3(1), dim3(64), 0, st, ticks);
    return hipGetLastError();
}

/* ------------------------------------------------- MoE h read-back */

/* Copies row r of the quantised SwiGLU activations (codes hc [rows, N],
 * scales hs as fp32 powers of two or E8M0 bytes [rows, N/128]) to row
 * pair_of_row[r] (identity when null) of codes / e8m0. One workgroup per
 * row; rows whose pair lies outside [0, rows) are skipped. */
__global__ __launch_bounds__(256) void apus_moe_h_gather_kernel(
    const uint8_t *__restrict__ hc, const void *__restrict__ hs, int hs_f32,
    const int32_t *__restrict__ pair_of_row, int rows, int N, uint8_t *__restrict__ codes,
    uint8_t *__restrict__ e8m0) {
    const int r = blockIdx.x;
    const int p = pair_of_row ? pair_of_row[r] : r;
    if ((unsigned)p >= (unsigned)rows) return;
    const int G = N >> 7;
    for (int i = threadIdx.x; i < N; i += 256) codes[(size_t)p * N + i] = hc[(size_t)r * N + i];
    for (int i = threadIdx.x; i < G; i += 256)
        e8m0[(size_t)p * G + i] = hs_f32 ? (uint8_t)apus_e8m0_of(((const float *)hs)[(size_t)r * G + i])
                                         : ((const uint8_t *)hs)[(size_t)r * G + i];
}

hipError_t apus_launch_moe_h_gather(const uint8_t *hc, const void *hs, int hs_f32,
                                    const int32_t *pair_of_row, int rows, int N, uint8_t *codes,
                                    uint8_t *e8m0, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (N % 128) return hipErrorInvalidValue;
    hipLaunchKernelGGL(apus_moe_h_gather_kernel, dim3(rows), dim3(256), 0, st, hc, hs, hs_f32,
                       pair_of_row, rows, N, codes, e8m0);
    return hipGetLastError();
}

/* ------------------------------------------------------------ SwiGLU */

/* h[i] = bf16(silu(min(g, L)) * clamp(u, +-L)) elementwise (c/moe.h:113-126):
 * the element function every fused MoE kernel applies, on its own. */
__global__ __launch_bounds__(256) void apus_swiglu_kernel(const float *__restrict__ g,
                                                          const float *__restrict__ u, size_t n,
                                                          float limit, float *__restrict__ h) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) h[i] = apus_swiglu_h(g[i], u[i], limit);
}

hipError_t apus_launch_swiglu(const float *g, const float *u, size_t n, float limit, float *h,
                              hipStream_t st) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(apus_swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, g, u,
                       n, limit, h);
    return hipGetLastError();
}
