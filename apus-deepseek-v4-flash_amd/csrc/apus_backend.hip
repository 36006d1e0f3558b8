/*
 * apus_backend.hip — C-ABI host side of the MI355X backend (include/apus_hip.h).
 *
 * Mirrors the structure of apus's Metal backend (c/backend_metal.mm:660-746):
 * lazy device init, a hook table filled by enable, weight caches for the
 * dense linears keyed by host pointer, per-op fail-soft (nonzero return =
 * caller runs its CPU kernel). Differences that follow from MI355X:
 *  - weights are copied once into HBM (discrete memory, no zero-copy);
 *  - routed experts are cached by (layer, expert id) in an HBM-resident
 *    store instead of by pointer, so evicted/reused host slabs never alias;
 *  - everything runs on one HIP stream; host-pointer entry points stage
 *    through device scratch and synchronise before returning.
 */
#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <fcntl.h>
#include <unistd.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <condition_variable>
#include <deque>
#include <mutex>
#include <thread>
#include <unordered_map>
#include <vector>

#include "../../include/apus_hip.h"
#include "apus_container.h"
#include "apus_internal.h"
#include "apus_numerics.h"

/* ------------------------------------------------------------------ state */

/* Workspace of the allocation-free routed dispatch
 * (apus_hip_moe_routed_dev_noalloc): one statically sized array in device
 * memory, which every GPU the library runs on holds until the process ends.
 * In host code the name is only a stand-in: its device address comes from
 * hipGetSymbolAddress at initialisation (per device) and only that address
 * is ever passed to kernels. */
#define APUS_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
static __device__ __align__(256) uint8_t scratch[APUS_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local char g_err[512];

void set_err(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}

struct DevBuf {
    void *p = nullptr;
    size_t n = 0;
};

struct DenseW {        /* one cached dense weight (codes/packed + scales) */
    const void *host_scales;
    uint8_t *w, *ws;
    size_t wbytes, sbytes;
    uint64_t fp;
    int wfmt, O, K;    /* the layout of a tiled copy depends on the shape */
    bool tiled;        /* held in the MFMA-tiled layout */
};

struct ExpertW {       /* one cached routed expert, six tensors */
    uint8_t *p[6];
    size_t bytes;
    int dim, inter;    /* a (layer, id) reused with another shape is re-uploaded */
    bool tiled;
    uint64_t fp;       /* fingerprint of the six host tensors' bytes (not their addresses) */
};

struct State {
    bool enabled = false;
    bool inited = false;
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
    /* concurrency lanes for the *_dev entry points: lane 0 is `stream` */
    hipStream_t lane[8] = {};
    hipEvent_t lane_ev[8] = {};
    int nlanes = 1, cur_lane = 0;
    /* the MoE sublayer's shared expert runs beside the router and the routed
     * experts on this stream (forked from and joined to the caller's) */
    hipStream_t side = nullptr;
    hipEvent_t side_fork = nullptr, side_done = nullptr;
    /* per-lane counters of the one-token MoE h hand-off (apus_moe_pair13):
     * zeroed once here, every launch leaves them zero */
    unsigned *pair_tk[8] = {};
    /* grid barrier words of the one-launch one-token layer
     * (apus_moe_layer1_kernel), which runs on lane 0 only: two of those
     * launches running at once would each wait for CUs the other holds */
    unsigned *layer_bar = nullptr;
    bool layer1 = false, layer1_ok = false;
    /* set to 1 by a layer workgroup whose barrier wait gave up (pinned host
     * memory, written by the kernel through l1_flag_dev); finish() reports
     * it as an error */
    volatile unsigned *l1_flag = nullptr;
    unsigned *l1_flag_dev = nullptr;
    unsigned l1_spin = 1u << 23;
    unsigned l1_faults = 0;       /* workgroups that gave up, seen by finish() since the last read */
    std::unordered_map<const void *, DenseW> dense;
    std::unordered_map<uint64_t, ExpertW> experts;
    DevBuf slots[8];          /* grow-only device scratch of the host-pointer calls */
    /* pinned staging of the host-pointer calls' small transfers (x, out,
     * ids, ...): filled from offset 0 after every finish(), so a region is
     * never rewritten before the copy that reads it has run; downloads land
     * here and are copied to the caller's buffers after the sync */
    uint8_t *pin = nullptr;
    uint8_t *pin_dev = nullptr;   /* the buffer's device address (kernels write results there) */
    size_t pin_used = 0;
    bool pin_failed = false;
    std::vector<std::pair<void *, size_t>> pin_out;   /* (caller dst, bytes) per staged download */
    std::vector<size_t> pin_out_off;
    /* device address of `scratch` per device ordinal (this backend runs on
     * device 0) */
    uint8_t *noalloc_scratch[16] = {};
    uint64_t bytes_uploaded = 0, bytes_resident = 0, dispatches = 0;
    size_t dense_budget = 0;
    ApusHipHooks hooks{};
};

State g;
std::mutex g_mu;

bool ok(hipError_t e, const char *what) {
    if (e == hipSuccess) return true;
    set_err("%s: %s", what, hipGetErrorString(e));
    return false;
}

/* counters per lane: (pairs + tokens) x (inter / 128) groups */
constexpr size_t PAIR_TK_CAP = 8192;

bool alloc_pair_tickets(int lane) {
    if (g.pair_tk[lane]) return true;
    void *p = nullptr;
    if (!ok(hipMalloc(&p, PAIR_TK_CAP * sizeof(unsigned)), "hipMalloc tickets") ||
        !ok(hipMemset(p, 0, PAIR_TK_CAP * sizeof(unsigned)), "hipMemset tickets"))
        return false;
    g.pair_tk[lane] = (unsigned *)p;
    return true;
}

void pin_reset();

bool ensure_init() {
    if (g.inited) {
        pin_reset();
        return true;
    }
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        set_err("no HIP device visible");
        return false;
    }
    hipDeviceProp_t prop;
    if (!ok(hipGetDeviceProperties(&prop, 0), "hipGetDeviceProperties")) return false;
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        set_err("device 0 is %s, this backend is built for gfx950 only", prop.gcnArchName);
        return false;
    }
    if (!ok(hipSetDevice(0), "hipSetDevice")) return false;
    {
        void *p = nullptr;
        if (!ok(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)") || !p)
            return false;
        g.noalloc_scratch[0] = (uint8_t *)p;
    }
    if (!ok(hipStreamCreateWithFlags(&g.stream, hipStreamNonBlocking), "hipStreamCreate")) return false;
    if (!ok(hipEventCreate(&g.ev0), "hipEventCreate")) return false;
    if (!ok(hipEventCreate(&g.ev1), "hipEventCreate")) return false;
    g.lane[0] = g.stream;
    if (!ok(hipEventCreateWithFlags(&g.lane_ev[0], hipEventDisableTiming), "hipEventCreate")) return false;
    if (!alloc_pair_tickets(0)) return false;
    {
        void *p = nullptr;
        const size_t nb = (size_t)apus_moe_layer1_bar_words() * sizeof(unsigned);
        if (!ok(hipMalloc(&p, nb), "hipMalloc layer barrier") ||
            !ok(hipMemset(p, 0, nb), "hipMemset layer barrier"))
            return false;
        g.layer_bar = (unsigned *)p;
        void *hf = nullptr, *hd = nullptr;
        if (!ok(hipHostMalloc(&hf, 256, hipHostMallocMapped | hipHostMallocCoherent), "hipHostMalloc layer flag") ||
            !ok(hipHostGetDevicePointer(&hd, hf, 0), "hipHostGetDevicePointer layer flag"))
            return false;
        *(volatile unsigned *)hf = 0;
        g.l1_flag = (volatile unsigned *)hf;
        g.l1_flag_dev = (unsigned *)hd;
        /* the one-launch layer needs its 256 workgroups resident together;
         * APUS_HIP_LAYER1=0 turns it off (two launches per layer) */
        const char *v = getenv("APUS_HIP_LAYER1");
        g.layer1_ok = prop.multiProcessorCount >= 256 && apus_moe_layer1_fits() >= 1;
        g.layer1 = g.layer1_ok && !(v && atoi(v) == 0);
    }
    if (!ok(hipStreamCreateWithFlags(&g.side, hipStreamNonBlocking), "hipStreamCreate") ||
        !ok(hipEventCreateWithFlags(&g.side_fork, hipEventDisableTiming), "hipEventCreate") ||
        !ok(hipEventCreateWithFlags(&g.side_done, hipEventDisableTiming), "hipEventCreate"))
        return false;
    const char *mb = getenv("APUS_HIP_DENSE_MB");
    g.dense_budget = (size_t)(mb ? strtoull(mb, nullptr, 10) : 131072ull) << 20;
    g.inited = true;
    return true;
}

/* grow-only device scratch slot i of at least n bytes */
void *scratch_slot(int i, size_t n) {
    DevBuf &b = g.slots[i];
    if (b.n >= n && b.p) return b.p;
    if (b.p) { (void)hipStreamSynchronize(g.stream); (void)hipFree(b.p); b.p = nullptr; b.n = 0; }
    size_t want = n < 4096 ? 4096 : n;
    if (!ok(hipMalloc(&b.p, want), "hipMalloc scratch")) return nullptr;
    b.n = want;
    return b.p;
}

/* stream of the currently selected lane (for *_dev launches) */
hipStream_t dev_stream() { return g.lane[g.cur_lane]; }

/* the h hand-off counters of the lane that owns stream st */
unsigned *pair_tickets(hipStream_t st) {
    for (int i = 0; i < g.nlanes; i++)
        if (g.lane[i] == st) return g.pair_tk[i];
    return g.pair_tk[0];
}

constexpr size_t PIN_CAP = (size_t)8 << 20;     /* pinned staging bytes */
constexpr size_t PIN_SMALL = (size_t)1 << 20;   /* transfers up to this size are staged */

/* a 256-aligned region of the pinned staging buffer, or null (then the
 * transfer goes straight from or to pageable memory) */
uint8_t *pin_take(size_t n) {
    if (n > PIN_SMALL || g.pin_failed) return nullptr;
    if (!g.pin) {
        if (hipHostMalloc((void **)&g.pin, PIN_CAP, hipHostMallocDefault) != hipSuccess) {
            (void)hipGetLastError();
            g.pin = nullptr;
            g.pin_failed = true;
            return nullptr;
        }
    }
    const size_t off = (g.pin_used + 255) & ~(size_t)255;
    if (off + n > PIN_CAP) return nullptr;
    g.pin_used = off + n;
    return g.pin + off;
}

/* a device-visible region of the staging buffer for a call's result: the
 * last kernel writes it there (no download copy) and it reaches dst at
 * finish(); null when staging is not available (then download as usual) */
void *out_direct(void *dst, size_t n) {
    if (!dst || n > PIN_SMALL || g.pin_failed) return nullptr;
    const size_t used0 = g.pin_used;
    uint8_t *p = pin_take(n);
    if (!p) return nullptr;
    if (!g.pin_dev) {
        void *d = nullptr;
        if (hipHostGetDevicePointer(&d, g.pin, 0) != hipSuccess || !d) {
            (void)hipGetLastError();
            g.pin_used = used0;
            return nullptr;
        }
        g.pin_dev = (uint8_t *)d;
    }
    g.pin_out.emplace_back(dst, n);
    g.pin_out_off.push_back((size_t)(p - g.pin));
    return g.pin_dev + (p - g.pin);
}

bool upload(void *dst, const void *src, size_t n) {
    if (uint8_t *p = pin_take(n)) {
        memcpy(p, src, n);
        return ok(hipMemcpyAsync(dst, p, n, hipMemcpyHostToDevice, g.stream), "H2D");
    }
    return ok(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, g.stream), "H2D");
}

bool download(void *dst, const void *src, size_t n) {
    if (uint8_t *p = pin_take(n)) {
        g.pin_out.emplace_back(dst, n);
        g.pin_out_off.push_back((size_t)(p - g.pin));
        return ok(hipMemcpyAsync(p, src, n, hipMemcpyDeviceToHost, g.stream), "D2H");
    }
    return ok(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, g.stream), "D2H");
}

/* at the start of a call: staging left over by a call that failed before
 * its finish() is dropped once the stream has drained (its downloads never
 * reach the caller that gave up on them). Skipped while the stream is being
 * captured (no host call is in flight then). */
void pin_reset() {
    if (g.pin_used == 0 && g.pin_out.empty()) return;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(g.stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return;
    (void)hipStreamSynchronize(g.stream);
    g.pin_out.clear();
    g.pin_out_off.clear();
    g.pin_used = 0;
}

/* After lane 0 has drained: if a one-launch layer's barrier wait gave up
 * since the last check, fold its fault count into g.l1_faults, reset the
 * barrier words and report an error (the launch wrote NaN into the y
 * columns of every workgroup that gave up). */
bool l1_fault_check() {
    if (!g.l1_flag || !*g.l1_flag) return true;
    *g.l1_flag = 0;
    unsigned n = 0;
    const size_t nb = (size_t)apus_moe_layer1_bar_words() * sizeof(unsigned);
    if (!ok(hipMemcpy(&n, g.layer_bar + apus_moe_layer1_fault_word(), sizeof(unsigned),
                      hipMemcpyDeviceToHost), "hipMemcpy layer1 faults") ||
        !ok(hipMemset(g.layer_bar, 0, nb), "hipMemset layer barrier") ||
        !ok(hipDeviceSynchronize(), "hipDeviceSynchronize"))
        return false;
    g.l1_faults += n;
    set_err("one-launch layer: %u workgroup(s) gave up waiting at the grid barrier (another kernel or "
            "process held CUs); their y columns are NaN: rerun with apus_hip_layer1(0)", n);
    return false;
}

/* wait for the stream, then hand staged downloads to their callers' buffers
 * and release the staging buffer; false (with the error set) if the stream
 * failed or a one-launch layer gave up at its barrier */
bool finish() {
    bool r = ok(hipStreamSynchronize(g.stream), "hipStreamSynchronize");
    if (r) r = l1_fault_check();
    if (r) {
        for (size_t i = 0; i < g.pin_out.size(); ++i)
            memcpy(g.pin_out[i].first, g.pin + g.pin_out_off[i], g.pin_out[i].second);
    }
    g.pin_out.clear();
    g.pin_out_off.clear();
    g.pin_used = 0;
    return r;
}

bool launched(hipError_t e, const char *what) {
    g.dispatches++;
    return ok(e, what);
}

/* 64-bit fingerprint of 16 words sampled across a host buffer (cheap; makes a
 * freed-and-reused host address with new contents re-upload instead of
 * silently reading the stale device copy) */
uint64_t fingerprint(const uint8_t *p, size_t n) {
    uint64_t h = 0xcbf29ce484222325ull ^ n;
    for (int i = 0; i < 16; i++) {
        uint64_t v = 0;
        const size_t off = (n > 8) ? (size_t)((n - 8) * (uint64_t)i / 15) : 0;
        memcpy(&v, p + off, n >= 8 ? 8 : n);
        h = (h ^ v) * 0x100000001b3ull;
    }
    return h;
}

/* dense weight cache lookup/insert, keyed by the host weight pointer (the
 * engine's weight pointers are stable, c/backend_metal.h:38-43); a hit whose
 * format, shape (O, K: the tiled layout depends on it), scale pointer or
 * sampled contents changed is re-uploaded */
/* shapes whose weights are kept in the MFMA-tiled layout (the decode,
 * prefill and tile schedules read it) */
bool tiled_shape(int O, int K) { return apus_fast_k(K) && O > 0 && O % 128 == 0; }

/* routed experts of this shape are held MFMA-tiled (w1/w3 [inter, dim] and
 * w2 [dim, inter] with K 2048 or 4096: the grouped schedules) */
bool moe_tiled(int dim, int inter) {
    return apus_group_k(dim) && apus_group_k(inter) && inter % 128 == 0 && dim % 128 == 0;
}

/* host row-major weights -> device, MFMA-tiled when `tiled` (staged through
 * scratch slots 4 and 5) */
bool upload_weights(int wfmt, uint8_t *dw, uint8_t *dws, const void *w, const void *ws,
                    size_t wbytes, size_t sbytes, int O, int K, bool tiled) {
    if (!tiled) return upload(dw, w, wbytes) && upload(dws, ws, sbytes);
    uint8_t *sw = (uint8_t *)scratch_slot(4, wbytes);
    uint8_t *ss = (uint8_t *)scratch_slot(5, sbytes);
    if (!sw || !ss || !upload(sw, w, wbytes) || !upload(ss, ws, sbytes)) return false;
    if (!launched(apus_launch_pack(wfmt, sw, ss, dw, dws, O, K, 0, g.stream), "pack")) return false;
    if (wfmt == APUS_W_FP8 && !ok(hipMemcpyAsync(dws, ss, sbytes, hipMemcpyDeviceToDevice, g.stream),
                                  "D2D scales"))
        return false;
    /* the staging slots are reused by the next upload */
    return finish();
}

/* ---- input domain of the host-pointer entry points. The matrix cores
 * read E8M0 byte 255 and E4M3 codes 0x7F / 0xFF as NaN, where the reference
 * decodes +inf and +-480 (c/fp4.h:209-217, :255-260); a non-finite
 * activation makes the reference's group scale +inf (c/fp4.h:300-317). Such
 * inputs are refused (nonzero: the caller runs its CPU kernel, which gives
 * the reference's result); the *_dev entry points document them as outside
 * their contract instead (a row with a non-finite activation comes out NaN). */
bool x_finite(const float *x, size_t n, const char *what) {
    const uint32_t *u = (const uint32_t *)x;
    for (size_t i = 0; i < n; i++)
        if ((u[i] & 0x7f800000u) == 0x7f800000u) {
            set_err("%s: non-finite activation at element %zu (outside the GPU contract; "
                    "the CPU kernel handles it)", what, i);
            return false;
        }
    return true;
}

bool e8m0_ok(const uint8_t *s, size_t n, const char *what) {
    if (n && memchr(s, 0xff, n)) {
        set_err("%s: E8M0 scale byte 255 (+inf in the reference, NaN on the matrix cores)", what);
        return false;
    }
    return true;
}

bool e4m3_ok(const uint8_t *c, size_t n, const char *what) {
    for (size_t i = 0; i < n; i++)
        if ((c[i] & 0x7f) == 0x7f) {
            set_err("%s: E4M3 code %#x at %zu (+-480 in the reference, NaN on the matrix cores)",
                    what, c[i], i);
            return false;
        }
    return true;
}

/* activation scales of pre-quantised rows: finite powers of two */
bool pow2_ok(const float *s, size_t n, const char *what) {
    const uint32_t *u = (const uint32_t *)s;
    for (size_t i = 0; i < n; i++) {
        const uint32_t e = (u[i] >> 23) & 0xffu;
        if ((u[i] & 0x807fffffu) || e == 0 || e == 0xffu) {
            set_err("%s: activation scale %zu is not a positive finite power of two", what, i);
            return false;
        }
    }
    return true;
}

/* the stored weight bytes the matrix cores decode as the reference does */
bool weights_ok(int wfmt, const uint8_t *w, const uint8_t *ws, size_t wbytes, size_t sbytes,
                const char *what) {
    if (wfmt == APUS_W_FP8 && !e4m3_ok(w, wbytes, what)) return false;
    return wfmt > APUS_W_FP8 || e8m0_ok(ws, sbytes, what);
}

const DenseW *dense_weight(int wfmt, const uint8_t *w, const uint8_t *ws, size_t wbytes,
                           size_t sbytes, int O, int K) {
    const uint64_t fp = fingerprint(w, wbytes) ^ (ws && sbytes ? fingerprint(ws, sbytes) * 31 : 0);
    auto it = g.dense.find(w);
    if (it != g.dense.end()) {
        DenseW &d = it->second;
        if (d.host_scales == ws && d.wbytes == wbytes && d.sbytes == sbytes && d.fp == fp &&
            d.wfmt == wfmt && d.O == O && d.K == K)
            return &d;
        (void)hipStreamSynchronize(g.stream);
        (void)hipFree(d.w);
        (void)hipFree(d.ws);
        g.bytes_resident -= d.wbytes + d.sbytes;
        g.dense.erase(it);
    }
    if (g.bytes_resident + wbytes + sbytes > g.dense_budget) {
        set_err("dense weight budget exhausted (APUS_HIP_DENSE_MB)");
        return nullptr;
    }
    if (!weights_ok(wfmt, w, ws, wbytes, sbytes, "weight upload")) return nullptr;
    DenseW d{ws, nullptr, nullptr, wbytes, sbytes, fp, wfmt, O, K, false};
    if (!ok(hipMalloc(&d.w, wbytes), "hipMalloc weight")) return nullptr;
    if (!ok(hipMalloc(&d.ws, sbytes), "hipMalloc scales")) { (void)hipFree(d.w); return nullptr; }
    d.tiled = wfmt <= APUS_W_FP8 && tiled_shape(O, K);
    if (!upload_weights(wfmt, d.w, d.ws, w, ws, wbytes, sbytes, O, K, d.tiled)) {
        (void)hipFree(d.w); (void)hipFree(d.ws);
        return nullptr;
    }
    g.bytes_uploaded += wbytes + sbytes;
    g.bytes_resident += wbytes + sbytes;
    return &(g.dense[w] = d);
}

bool shape_ok(int M, int K, int O) {
    if (M <= 0 || O <= 0 || K <= 0 || (K % 128) != 0) {
        set_err("unsupported shape M=%d K=%d O=%d (needs K %% 128 == 0)", M, K, O);
        return false;
    }
    return true;
}

/* wfmt may carry APUS_HIP_W_TILED */
int gemm_dev(int wfmt, const uint8_t *w, const uint8_t *ws, const uint8_t *acodes,
             const float *as, float *out, int M, int O, int K, int round_out, hipStream_t st) {
    ApusGemmArgs a{};
    a.wtiled = (wfmt & APUS_HIP_W_TILED) ? 1 : 0;
    wfmt &= ~APUS_HIP_W_TILED;
    a.acodes = acodes; a.ascale = as; a.ents = nullptr;
    a.ent0.w = w; a.ent0.ws = ws; a.ent0.out = out;
    a.ent0.arows = nullptr; a.ent0.orows = nullptr;
    a.ent0.a0 = 0; a.ent0.o0 = 0; a.ent0.M = M;
    a.O = O; a.K = K; a.ldo = O; a.round_out = round_out;
    return launched(apus_launch_gemm(wfmt, &a, 1, st), "gemm") ? 0 : 1;
}

/* fp32 x -> BF16 out linear in one launch when M <= 8 and the shape has a
 * few-row schedule (the act quant runs in the GEMM's staging); returns -1
 * when the shape does not qualify (the caller quantises, then multiplies) */
int linear_fused(int wfmt, const uint8_t *w, const uint8_t *ws, const float *x, float *out,
                 int M, int K, int O, hipStream_t st) {
    if (M > 8 || !apus_fast_k(K) || O % 128) return -1;
    ApusGemmArgs a{};
    a.wtiled = (wfmt & APUS_HIP_W_TILED) ? 1 : 0;
    wfmt &= ~APUS_HIP_W_TILED;
    a.ents = nullptr;
    a.ent0.w = w; a.ent0.ws = ws; a.ent0.out = out;
    a.ent0.arows = nullptr; a.ent0.orows = nullptr;
    a.ent0.a0 = 0; a.ent0.o0 = 0; a.ent0.M = M;
    a.O = O; a.K = K; a.ldo = O; a.round_out = 1;
    a.asrc = APUS_A_F32; a.ax = x;
    return launched(apus_launch_gemm_few(wfmt, &a, 1, 8, 0, st), "linear") ? 0 : 1;
}

/* host-pointer linear: stage x, quantise, GEMM, BF16 out, copy back */
int linear_host(int wfmt, const uint8_t *w, const uint8_t *ws, const float *x,
                float *out, int M, int K, int O) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!ensure_init() || !shape_ok(M, K, O)) return 1;
    const size_t wbytes = wfmt == APUS_W_FP4 ? (size_t)O * K / 2 : (size_t)O * K;
    const size_t sbytes = wfmt == APUS_W_FP4 ? (size_t)O * K / 32
                                             : (size_t)((O + 127) / 128) * (K / 128);
    if (!x_finite(x, (size_t)M * K, "linear")) return 1;
    const DenseW *d = dense_weight(wfmt, w, ws, wbytes, sbytes, O, K);
    if (!d) return 1;
    const int wf = wfmt | (d->tiled ? APUS_HIP_W_TILED : 0);
    const size_t nab = K / 128;
    float *dx = (float *)scratch_slot(0, (size_t)M * K * 4);
    uint8_t *dc = (uint8_t *)scratch_slot(1, (size_t)M * K);
    float *dsc = (float *)scratch_slot(2, (size_t)M * nab * 4);
    float *dout = (float *)out_direct(out, (size_t)M * O * 4);
    const bool direct = dout != nullptr;
    if (!direct) dout = (float *)scratch_slot(3, (size_t)M * O * 4);
    if (!dx || !dc || !dsc || !dout) return 1;
    if (!upload(dx, x, (size_t)M * K * 4)) return 1;
    const int f = linear_fused(wf, d->w, d->ws, dx, dout, M, K, O, g.stream);
    if (f > 0) return 1;
    if (f < 0) {
        if (!launched(apus_launch_act_quant(dx, K, nullptr, M, K, dc, dsc, g.stream), "act_quant")) return 1;
        if (gemm_dev(wf, d->w, d->ws, dc, dsc, dout, M, O, K, 1, g.stream)) return 1;
    }
    if ((!direct && !download(out, dout, (size_t)M * O * 4)) || !finish()) return 1;
    return 0;
}

int gemm_host(int wfmt, const uint8_t *w, const uint8_t *ws, const uint8_t *acodes,
              const float *as, float *out, int M, int O, int K) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!ensure_init() || !shape_ok(M, K, O)) return 1;
    const size_t wbytes = wfmt == APUS_W_FP4 ? (size_t)O * K / 2 : (size_t)O * K;
    const size_t sbytes = wfmt == APUS_W_FP4 ? (size_t)O * K / 32
                                             : (size_t)((O + 127) / 128) * (K / 128);
    const size_t nab = K / 128;
    if (!weights_ok(wfmt, w, ws, wbytes, sbytes, "gemm") || !e4m3_ok(acodes, (size_t)M * K, "gemm") ||
        !pow2_ok(as, (size_t)M * nab, "gemm"))
        return 1;
    uint8_t *dw = (uint8_t *)scratch_slot(4, wbytes);
    uint8_t *dws = (uint8_t *)scratch_slot(5, sbytes);
    uint8_t *dc = (uint8_t *)scratch_slot(1, (size_t)M * K);
    float *dsc = (float *)scratch_slot(2, (size_t)M * nab * 4);
    float *dout = (float *)scratch_slot(3, (size_t)M * O * 4);
    if (!dw || !dws || !dc || !dsc || !dout) return 1;
    if (!upload(dw, w, wbytes) || !upload(dws, ws, sbytes) ||
        !upload(dc, acodes, (size_t)M * K) || !upload(dsc, as, (size_t)M * nab * 4))
        return 1;
    if (gemm_dev(wfmt, dw, dws, dc, dsc, dout, M, O, K, 0, g.stream)) return 1;
    if (!download(out, dout, (size_t)M * O * 4) || !finish()) return 1;
    return 0;
}

/* workspace carve-up for the routed dispatch */
struct MoeWs {
    uint8_t *xc; float *xs;
    int32_t *pair, *tok;
    ApusGemmEnt *e13s, *e2s, *e13l, *e2l;   /* few-row and many-row expert tables */
    float *gm, *um; uint8_t *hc; float *hs; float *eo;
    uint8_t **tab;
    unsigned *tickets;   /* one per 16 output columns of w2 */
    int2 *items13, *items2;   /* many-row work lists */
    int n_items;
    size_t total;
};

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

/* experts with at most this many routed pairs take the few-row schedule */
constexpr int MOE_SMALL = 8;

MoeWs moe_carve(void *base, int s, int topk, int E, int dim, int inter) {
    MoeWs w{};
    const size_t nj = (size_t)s * topk;
    size_t off = 0;
    auto take = [&](size_t n) { size_t o = off; off += align256(n); return o; };
    size_t o_xc = take((size_t)s * dim), o_xs = take((size_t)s * (dim / 128) * 4);
    size_t o_pair = take(nj * 4), o_tok = take(nj * 4);
    const size_t te = (size_t)E * sizeof(ApusGemmEnt);
    size_t o_e13s = take(2 * te), o_e2s = take(te), o_e13l = take(2 * te), o_e2l = take(te);
    size_t o_g = take((nj + s) * inter * 4), o_u = take(nj * inter * 4);
    size_t o_hc = take((nj + s) * inter), o_hs = take((nj + s) * (inter / 128) * 4);
    size_t o_eo = take(nj * dim * 4);
    size_t o_tab = take(6 * (size_t)E * sizeof(void *));
    size_t o_tk = take((size_t)(dim / 16) * sizeof(unsigned));
    const int n_items = apus_moe_items_bound((int)nj, E, MOE_SMALL);
    size_t o_i13 = take(2 * (size_t)n_items * sizeof(int2)), o_i2 = take((size_t)n_items * sizeof(int2));
    w.n_items = n_items;
    w.total = off;
    if (base) {
        uint8_t *b = (uint8_t *)base;
        w.xc = b + o_xc; w.xs = (float *)(b + o_xs);
        w.pair = (int32_t *)(b + o_pair); w.tok = (int32_t *)(b + o_tok);
        w.e13s = (ApusGemmEnt *)(b + o_e13s); w.e2s = (ApusGemmEnt *)(b + o_e2s);
        w.e13l = (ApusGemmEnt *)(b + o_e13l); w.e2l = (ApusGemmEnt *)(b + o_e2l);
        w.gm = (float *)(b + o_g); w.um = (float *)(b + o_u);
        w.hc = b + o_hc; w.hs = (float *)(b + o_hs); w.eo = (float *)(b + o_eo);
        w.tab = (uint8_t **)(b + o_tab);
        w.tickets = (unsigned *)(b + o_tk);
        w.items13 = (int2 *)(b + o_i13);
        w.items2 = (int2 *)(b + o_i2);
    }
    return w;
}

/* routed pairs up to which the dispatch runs per pair (APUS_HIP_MOE_PAIRS
 * overrides; 0 = always sort by expert) */
int moe_pair_max() {
    static const int v = [] {
        const char *e = getenv("APUS_HIP_MOE_PAIRS");
        return e ? atoi(e) : 32;
    }();
    return v;
}

/* the routed-dispatch pipeline on device data; tab = 6 device arrays of E
 * pointers (w1, w1s, w2, w2s, w3, w3s) */
/* regularly spaced expert slabs (an expert store layer): tensor i of expert
 * e at base + e * stride + off[i], i = w1, w1s, w2, w2s, w3, w3s */
struct MoeSlab {
    const uint8_t *base;
    size_t stride, off[6];
};

/* whether moe_pipeline runs the one-token kernels with the FP8 shared expert
 * fused in (its w2 needs K = inter = 2048) */
bool moe_pair_mode(int dim, int inter, int s, int topk) {
    return s * topk <= moe_pair_max() && (dim == 2048 || dim == 4096) &&
           (inter == 2048 || inter == 4096) && (topk == 6 || topk == 8);
}
bool moe_pair_fused(int dim, int inter, int s, int topk) {
    return moe_pair_mode(dim, inter, s, topk) && inter == 2048;
}

/* expert choice fused into the one-token w1/w3 kernel (pair mode only) */
struct RouteFuse {
    const float *sel, *sp;         /* [s, E] selection and router scores */
    const int64_t *t2e, *ids;      /* hash routing (t2e set) */
    float scale;
    int E;
};

/* the FP8 shared expert fused into the one-token MoE kernels */
struct SharedFuse {
    const uint8_t *w[3], *ws[3];   /* w1, w2, w3 and their tile scales */
    int tiled;
    float *sh_out, *out;           /* sh = bf16(w2 h); out = bf16(y + sh) */
};

/* a dense FP8 linear of the same x co-scheduled in the one-token w1/w3
 * launch: out [s, 2 inter] = bf16(W x), W [2 inter, dim] */
struct DenseRider {
    const uint8_t *w, *ws;
    int tiled;
    float *out;
};

int moe_pipeline(int E, int dim, int inter, float limit, uint8_t *const *tab,
                 const float *x, const int32_t *idx, const float *wgt, int s,
                 int topk, float *y, const MoeWs &w, bool wtiled, const MoeSlab *slab,
                 hipStream_t st, const float *add_src = nullptr, float *add_out = nullptr,
                 hipEvent_t add_ready = nullptr, const SharedFuse *shf = nullptr,
                 const RouteFuse *rf = nullptr, const DenseRider *rd = nullptr) {
    /* with add_out: also add_out = bf16(y + add_src), fused into the last
     * launch where it can be; add_src is complete once add_ready has fired */
    auto wait_add = [&]() {
        return !add_ready || ok(hipStreamWaitEvent(st, add_ready, 0), "hipStreamWaitEvent");
    };
    const int nj = s * topk;
    ApusExpertTable t;
    t.w1 = tab; t.w1s = tab + E; t.w2 = tab + 2 * E; t.w2s = tab + 3 * E;
    t.w3 = tab + 4 * E; t.w3s = tab + 5 * E;
    const bool pair_shape = nj <= moe_pair_max() && (dim == 2048 || dim == 4096) &&
                            (inter == 2048 || inter == 4096);
    /* few pairs (decode), topk 6 or 8: two launches, no sorting pass. w1/w3
     * per (16 rows, pair) with SwiGLU in the epilogue -> h rows; w2 per 16
     * output columns over each token's pairs, accumulating y in (t, j) order
     * inside the workgroup */
    if ((shf || rf) && !(pair_shape && (topk == 6 || topk == 8))) {
        set_err("moe pipeline: fused shared expert / routing need the one-token kernels");
        return 1;
    }
    if (pair_shape && (topk == 6 || topk == 8)) {
        if (shf && inter != 2048) return 1;         /* callers check moe_pair_fused() */
        ApusGemmArgs a{};
        a.npairs = nj; a.acc_s = s;
        if (rf) {
            /* idx / wgt are written by the w1/w3 launch */
            a.rsel = rf->sel; a.rsp = rf->sp; a.rt2e = rf->t2e; a.rids = rf->ids;
            a.rscale = rf->scale; a.rE = rf->E;
            a.ridx = const_cast<int32_t *>(idx); a.rwgt = const_cast<float *>(wgt);
        }
        if (shf) {
            for (int i = 0; i < 3; i++) { a.shw[i] = shf->w[i]; a.shws[i] = shf->ws[i]; }
            a.sh_tiled = shf->tiled;
        }
        a.wtiled = wtiled;
        a.O = inter; a.K = dim; a.ldo = inter;
        a.ax = x; a.limit = limit;
        a.pidx = idx; a.adiv = topk; a.pE = E;
        a.pw[0] = t.w1; a.pws[0] = t.w1s; a.pw[1] = t.w3; a.pws[1] = t.w3s;
        if (slab) {
            a.pbase = slab->base; a.pstride = slab->stride;
            a.pwoff[0] = slab->off[0]; a.psoff[0] = slab->off[1];
            a.pwoff[1] = slab->off[4]; a.psoff[1] = slab->off[5];
        }
        a.pout[0] = w.gm;                           /* h rows [nj (+ s), inter] */
        if ((size_t)(nj + s) * (inter / 128) > PAIR_TK_CAP) {
            set_err("moe pipeline: %d pairs exceed the one-token kernels' counters", nj);
            return 1;
        }
        a.hq = w.hc; a.hqs = (uint8_t *)w.hs; a.hq_tk = pair_tickets(st);
        if (rd) { a.rdw = rd->w; a.rdws = rd->ws; a.rdout = rd->out; a.rdtiled = rd->tiled; }
        ApusGemmArgs b{};
        b.wtiled = wtiled;
        b.O = dim; b.K = inter; b.ldo = dim;
        b.hq = w.hc; b.hqs = (uint8_t *)w.hs;
        b.pidx = idx; b.pE = E;
        b.pw[0] = t.w2; b.pws[0] = t.w2s;
        if (slab) {
            b.pbase = slab->base; b.pstride = slab->stride;
            b.pwoff[0] = slab->off[2]; b.psoff[0] = slab->off[3];
        }
        b.acc_w = wgt; b.acc_y = y; b.acc_topk = topk; b.acc_s = s;
        b.add_src = add_out ? add_src : nullptr; b.add_out = add_out;
        b.npairs = nj;
        if (shf) {
            for (int i = 0; i < 3; i++) { b.shw[i] = shf->w[i]; b.shws[i] = shf->ws[i]; }
            b.sh_tiled = shf->tiled; b.sh_out = shf->sh_out; b.add_out = shf->out;
        }
        if (g.layer1 && st == g.lane[0] && s == 1 && topk == 6 && dim == 4096 && inter == 2048 &&
            !shf && !rf) {
            /* one launch: w1/w3 (+ rider), a grid barrier, w2 */
            if (add_out && !wait_add()) return 1;
            return launched(apus_launch_moe_layer1(&a, &b, g.layer_bar, g.l1_flag_dev, g.l1_spin, st), "one-token layer") ? 0 : 1;
        }
        if (!launched(apus_launch_moe_pair13(&a, nj, st), "pair w1/w3")) return 1;
        if (add_out && !wait_add()) return 1;
        return launched(apus_launch_moe_pair2(&b, st), "pair w2") ? 0 : 1;
    }
    /* experts with at most SMALL pairs take the few-row GEMM schedule; at
     * most min(E, nj) experts are small and at most nj / (SMALL + 1) are
     * large, so the launches cover only that many table slots */
    constexpr int SMALL = MOE_SMALL;
    if (!launched(apus_launch_act_quant(x, dim, nullptr, s, dim, w.xc, w.xs, st), "act_quant"))
        return 1;
    if (rd) {
        /* the dense linear on the quantised x (its own launch here) */
        ApusGemmArgs d{};
        d.wtiled = rd->tiled;
        d.acodes = w.xc; d.ascale = w.xs;
        d.ent0.w = rd->w; d.ent0.ws = rd->ws; d.ent0.out = rd->out; d.ent0.M = s;
        d.O = 2 * inter; d.K = dim; d.ldo = 2 * inter; d.round_out = 1;
        if (!launched(apus_launch_gemm(APUS_W_FP8, &d, 1, st), "dense rider")) return 1;
    }
    if (!launched(apus_launch_moe_route(idx, nj, topk, E, t, w.gm, w.um, w.eo, w.pair, w.tok,
                                        w.e13s, w.e2s, w.e13l, w.e2l, SMALL, w.items13, w.items2,
                                        w.n_items, st), "moe_route"))
        return 1;
    const int n_small = std::min(E, nj), n_large = std::min(E, nj / (SMALL + 1));
    ApusGemmArgs a{};
    a.wtiled = wtiled;
    a.acodes = w.xc; a.ascale = w.xs;
    a.O = inter; a.K = dim; a.ldo = inter; a.round_out = 1;
    ApusGemmArgs b{};
    b.wtiled = wtiled;
    b.acodes = w.hc; b.ascale = w.hs;
    b.O = dim; b.K = inter; b.ldo = dim; b.round_out = 1;
    /* the many-row entries run from the route kernel's work list (one
     * APUS_PREFILL_ROWS-row chunk per launch row, balanced) where the
     * many-row schedule applies */
    const bool use_items = (dim == 2048 || dim == 4096) && (inter == 2048 || inter == 4096);
    /* at these shapes the grouped GEMMs keep the accumulation orders of the
     * one-token kernels (w1/w3: one chain over K; w2: four K-quarter chains
     * added in order), so every token's y is bit-identical to dispatching it
     * alone, whatever the batch around it (the reference's batched ==
     * per-token property, tests/m9b/test_m9b.c:1-20) */
    if (use_items) { a.kchain = 1; b.kchain = 4; }
    for (int pass = 0; pass < 2; ++pass) {
        const int n = pass ? n_large : n_small;
        if (!n) continue;
        a.ents = pass ? w.e13l : w.e13s;
        a.max_m = pass ? 0 : SMALL;
        a.min_m = pass ? SMALL : 0;
        a.items = pass && use_items ? w.items13 : nullptr;
        const int rows = pass && use_items ? 2 * w.n_items : 2 * n;
        if (!launched(apus_launch_gemm(APUS_W_FP4, &a, rows, st), "gemm w1/w3")) return 1;
    }
    if (!launched(apus_launch_swiglu_quant(w.gm, w.um, nj, inter, limit, w.hc, w.hs, st),
                  "swiglu_quant"))
        return 1;
    for (int pass = 0; pass < 2; ++pass) {
        const int n = pass ? n_large : n_small;
        if (!n) continue;
        b.ents = pass ? w.e2l : w.e2s;
        b.max_m = pass ? 0 : SMALL;
        b.min_m = pass ? SMALL : 0;
        b.items = pass && use_items ? w.items2 : nullptr;
        const int rows = pass && use_items ? w.n_items : n;
        if (!launched(apus_launch_gemm(APUS_W_FP4, &b, rows, st), "gemm w2")) return 1;
    }
    if (add_out && !wait_add()) return 1;
    if (!launched(apus_launch_moe_accum(w.eo, wgt, s, topk, dim, y, add_out ? add_src : nullptr,
                                        add_out, st), "moe_accum"))
        return 1;
    return 0;
}

/* true (with the error set) while a graph capture is open on the backend
 * stream or the selected lane */
bool capturing(const char *what) {
    for (hipStream_t st : {g.stream, dev_stream()}) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
            set_err("%s: not allowed while a graph capture is open", what);
            return true;
        }
    }
    return false;
}

}  // namespace

/* ---------------------------------------------------------- store type */

struct ApusHipStore {
    int L, E, dim, inter;
    bool tiled;            /* expert matrices held MFMA-tiled */
    size_t sz[6];          /* bytes of w1, w1s, w2, w2s, w3, w3s */
    size_t expert_bytes;   /* 256-aligned slab per expert */
    std::vector<uint8_t *> layer_base;   /* one allocation per layer */
    std::vector<uint8_t **> layer_tab;   /* device pointer tables, 6*E each */
};

/* ============================================================== C ABI */

extern "C" {

int apus_hip_enable(char *err, size_t errcap) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!ensure_init()) {
        if (err && errcap) snprintf(err, errcap, "%s", g_err);
        return -1;
    }
    g.hooks.fp8_linear = apus_hip_fp8_linear;
    g.hooks.f32_linear = apus_hip_f32_linear;
    g.hooks.head_gemv = apus_hip_head_gemv;
    g.hooks.fp4_linear = apus_hip_fp4_linear;
    g.hooks.fp4_gemm_grouped = apus_hip_fp4_gemm_grouped;
    g.hooks.moe_routed = apus_hip_moe_routed;
    g.enabled = true;
    return 0;
}

void apus_hip_disable(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g.inited) return;
    (void)hipStreamSynchronize(g.stream);
    for (auto &kv : g.dense) { (void)hipFree(kv.second.w); (void)hipFree(kv.second.ws); }
    g.dense.clear();
    for (auto &kv : g.experts) (void)hipFree(kv.second.p[0]);
    g.experts.clear();
    for (auto &b : g.slots) { if (b.p) (void)hipFree(b.p); b.p = nullptr; b.n = 0; }
    if (g.pin) (void)hipHostFree(g.pin);
    g.pin = nullptr;
    g.pin_dev = nullptr;
    g.pin_used = 0;
    g.pin_out.clear();
    g.pin_out_off.clear();
    g.bytes_resident = 0;
    g.hooks = ApusHipHooks{};
    g.enabled = false;
}

int apus_hip_is_enabled(void) { return g.enabled ? 1 : 0; }
const ApusHipHooks *apus_hip_hooks(void) { return &g.hooks; }
uint64_t apus_hip_bytes_uploaded(void) { return g.bytes_uploaded; }
uint64_t apus_hip_bytes_resident(void) { return g.bytes_resident; }
uint64_t apus_hip_dispatches(void) { return g.dispatches; }
const char *apus_hip_last_error(void) { return g_err; }

int apus_hip_fp8_linear(const ApusFp8W *w, const float *x, float *out, int M, int K, int O) {
    if (!w || w->O != O || w->K != K) { set_err("fp8_linear: weight shape mismatch"); return 1; }
    return linear_host(APUS_W_FP8, w->codes, w->scales, x, out, M, K, O);
}

int apus_hip_fp4_linear(const ApusFp4W *w, const float *x, float *out, int M, int K, int O) {
    if (!w || w->O != O || w->K != K) { set_err("fp4_linear: weight shape mismatch"); return 1; }
    return linear_host(APUS_W_FP4, w->packed, w->scales, x, out, M, K, O);
}

int apus_hip_act_quant(const float *x, int M, int K, uint8_t *codes, float *scales) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!ensure_init() || !shape_ok(M, K, 1) || !x_finite(x, (size_t)M * K, "act_quant")) return 1;
    const size_t nab = K / 128;
    float *dx = (float *)scratch_slot(0, (size_t)M * K * 4);
    uint8_t *dc = (uint8_t *)scratch_slot(1, (size_t)M * K);
    float *dsc = (float *)scratch_slot(2, (size_t)M * nab * 4);
    if (!dx || !dc || !dsc) return 1;
    if (!upload(dx, x, (size_t)M * K * 4)) return 1;
    if (!launched(apus_launch_act_quant(dx, K, nullptr, M, K, dc, dsc, g.stream), "act_quant")) return 1;
    if (!download(codes, dc, (size_t)M * K) || !download(scales, dsc, (size_t)M * nab * 4) || !finish())
        return 1;
    return 0;
}

int apus_hip_fp4_gemm(const uint8_t *w, const uint8_t *ws, const uint8_t *acodes,
                      const float *as, float *out, int M, int O, int K) {
    return gemm_host(APUS_W_FP4, w, ws, acodes, as, out, M, O, K);
}

int apus_hip_fp8_gemm(const uint8_t *w, const uint8_t *ws, const uint8_t *acodes,
                      const float *as, float *out, int M, int O, int K) {
    return gemm_host(APUS_W_FP8, w, ws, acodes, as, out, M, O, K);
}

/* ---- plain-weight linears (c/attn.h:600-666, c/model.h:638-647) ---- */

static int wlinear_host(const void *w, bool bf16, const float *x, float *out, int M, int K, int O,
                        int flags) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!ensure_init()) return 1;
    if (M <= 0 || K <= 0 || O <= 0 || K % 8) {
        set_err("plain-weight linear: unsupported shape M=%d K=%d O=%d (needs K %% 8 == 0)", M, K, O);
        return 1;
    }
    const size_t wbytes = (size_t)O * K * (bf16 ? 2 : 4);
    const DenseW *d = dense_weight(bf16 ? APUS_W_BF16 : APUS_W_F32, (const uint8_t *)w, nullptr,
                                   wbytes, 0, O, K);
    if (!d) return 1;
    float *dx = (float *)scratch_slot(0, (size_t)M * K * 4);
    float *dout = (float *)out_direct(out, (size_t)M * O * 4);
    const bool direct = dout != nullptr;
    if (!direct) dout = (float *)scratch_slot(3, (size_t)M * O * 4);
    if (!dx || !dout || !upload(dx, x, (size_t)M * K * 4)) return 1;
    if (!launched(apus_launch_wgemv(d->w, dx, dout, M, K, O, (flags & 3) | (bf16 ? 4 : 0), g.stream),
                  "wgemv"))
        return 1;
    return (direct || download(out, dout, (size_t)M * O * 4)) && finish() ? 0 : 1;
}

int apus_hip_f32_linear(const float *w, const float *x, float *out, int M, int K, int O,
                        int flags) {
    if (!w || !x || !out || (flags & ~7)) return 1;
    return wlinear_host(w, (flags & APUS_HIP_W_BF16) != 0, x, out, M, K, O, flags);
}

int apus_hip_head_gemv(const ApusStTensor *head, const float *x, float *out, int64_t O,
                       int64_t K) {
    if (!head || !x || !out || O <= 0 || K <= 0 || O > 0x7fffffff || K > 0x7fffffff) return 1;
    const bool bf16 = head->dtype == APUS_ST_BF16;
    if ((!bf16 && head->dtype != APUS_ST_F32) || head->ndim != 2 || head->shape[0] != O ||
        head->shape[1] != K || head->nbytes != (size_t)(O * K * (bf16 ? 2 : 4)) || !head->data) {
        set_err("head_gemv: needs a BF16 or F32 [O, K] view");
        return 1;
    }
    return wlinear_host(head->data, bf16, x, out, 1, (int)K, (int)O, 0);
}

int apus_hip_wlinear_dev(const void *w, const float *x, float *out, int M, int K, int O,
                         int flags) {
    if (!ensure_init()) return 1;
    if (!w || !x || !out || (flags & ~7) || M <= 0 || K <= 0 || O <= 0 || K % 8) {
        set_err("wlinear_dev: bad arguments (K %% 8 == 0 needed)");
        return 1;
    }
    return launched(apus_launch_wgemv(w, x, out, M, K, O, flags, dev_stream()), "wgemv") ? 0 : 1;
}

int apus_hip_fp4_gemm_grouped(const ApusFp4GemmEnt *ents, size_t n_ent, const uint8_t *acodes,
                              const float *as, size_t O, size_t K) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!ensure_init()) return 1;
    if (!n_ent) return 0;
    if (!shape_ok(1, (int)K, (int)O)) return 1;
    size_t rows = 0, outrows = 0, max_m = 0;
    for (size_t i = 0; i < n_ent; i++) {
        if (ents[i].m0 + ents[i].M > rows) rows = ents[i].m0 + ents[i].M;
        if (ents[i].M > max_m) max_m = ents[i].M;
        outrows += ents[i].M;
    }
    const size_t nab = K / 128;
    if (!e4m3_ok(acodes, rows * K, "grouped gemm") || !pow2_ok(as, rows * nab, "grouped gemm"))
        return 1;
    uint8_t *dc = (uint8_t *)scratch_slot(1, rows * K + 1);
    float *dsc = (float *)scratch_slot(2, rows * nab * 4 + 4);
    float *dout = (float *)scratch_slot(3, outrows * O * 4 + 4);
    ApusGemmEnt *dents = (ApusGemmEnt *)scratch_slot(6, n_ent * sizeof(ApusGemmEnt));
    if (!dc || !dsc || !dout || !dents) return 1;
    if (!upload(dc, acodes, rows * K) || !upload(dsc, as, rows * nab * 4)) return 1;
    std::vector<ApusGemmEnt> he(n_ent);
    size_t orow = 0;
    bool tiled = false;     /* same (O, K) for every entry: all tiled or none */
    for (size_t i = 0; i < n_ent; i++) {
        const DenseW *d = dense_weight(APUS_W_FP4, ents[i].w, ents[i].ws, O * K / 2, O * K / 32,
                                       (int)O, (int)K);
        if (!d) return 1;
        tiled = d->tiled;
        he[i] = ApusGemmEnt{d->w, d->ws, dout, nullptr, nullptr, (int32_t)ents[i].m0,
                            (int32_t)orow, (int32_t)ents[i].M, 0};
        orow += ents[i].M;
    }
    if (!upload(dents, he.data(), n_ent * sizeof(ApusGemmEnt))) return 1;
    ApusGemmArgs a{};
    a.acodes = dc; a.ascale = dsc; a.ents = dents;
    a.O = (int)O; a.K = (int)K; a.ldo = (int)O; a.round_out = 0; a.max_m = (int)max_m;
    a.wtiled = tiled ? 1 : 0;
    if (!launched(apus_launch_gemm(APUS_W_FP4, &a, (int)n_ent, g.stream), "grouped gemm")) return 1;
    orow = 0;
    for (size_t i = 0; i < n_ent; i++) {
        if (ents[i].M && !download(ents[i].out, dout + orow * O, ents[i].M * O * 4)) return 1;
        orow += ents[i].M;
    }
    return finish() ? 0 : 1;
}

int apus_hip_moe_routed(const ApusMoeW *w, const float *x, const int32_t *idx, const float *wgt,
                        int s, float *y) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!ensure_init()) return 1;
    if (!w || s <= 0) { set_err("moe_routed: bad arguments"); return 1; }
    const int E = w->E, topk = w->topk, dim = w->dim, inter = w->inter;
    if (E <= 0 || topk <= 0 || dim % 128 || inter % 128 || dim <= 0 || inter <= 0) {
        set_err("moe_routed: unsupported shape E=%d dim=%d inter=%d", E, dim, inter);
        return 1;
    }
    const int nj = s * topk;
    for (int q = 0; q < nj; q++)
        if (idx[q] < 0 || idx[q] >= E) { set_err("moe_routed: expert id out of range"); return 1; }
    if (!x_finite(x, (size_t)s * dim, "moe_routed")) return 1;
    /* resident expert slabs keyed by (layer, eid). As in c/moe.h:419-431,
     * a resolve hook gets one hint per unique routed expert (first-seen
     * order) before any weight is resolved; then every unique expert is
     * resolved (c/moe.h:439-441) before anything is uploaded or launched, so
     * a failing resolve returns nonzero with nothing issued. A resolved slab
     * may sit at another address on every call (the store's tiers move it);
     * the cached copy is kept while the bytes' fingerprint matches. */
    const size_t sz[6] = {(size_t)inter * dim / 2, (size_t)inter * dim / 32,
                          (size_t)dim * inter / 2, (size_t)dim * inter / 32,
                          (size_t)inter * dim / 2, (size_t)inter * dim / 32};
    std::vector<int> uniq;
    std::vector<char> seen((size_t)E, 0);
    for (int q = 0; q < nj; q++)
        if (!seen[idx[q]]) { seen[idx[q]] = 1; uniq.push_back(idx[q]); }
    if (w->hook_resolve && w->hook_hint)
        for (int e : uniq) w->hook_hint(w->hook_hint_ctx ? w->hook_hint_ctx : w->hook_ctx, w->layer_id, e);
    std::vector<std::array<const void *, 6>> srcs(uniq.size());
    for (size_t u = 0; u < uniq.size(); u++) {
        const int e = uniq[u];
        ApusFp4W r1, r2, r3;
        if (w->hook_resolve) {
            if (w->hook_resolve(w->hook_ctx, w->layer_id, e, &r1, &r2, &r3)) {
                set_err("moe_routed: expert resolve failed (layer %d, expert %d)", w->layer_id, e);
                return 1;
            }
        } else {
            r1 = w->w1[e]; r2 = w->w2[e]; r3 = w->w3[e];
        }
        srcs[u] = {r1.packed, r1.scales, r2.packed, r2.scales, r3.packed, r3.scales};
        for (int i = 0; i < 6; i++)
            if (!srcs[u][i]) {
                set_err("moe_routed: expert %d of layer %d has a null tensor", e, w->layer_id);
                return 1;
            }
        for (int i = 1; i < 6; i += 2)
            if (!e8m0_ok((const uint8_t *)srcs[u][i], sz[i], "moe_routed expert")) return 1;
    }
    std::vector<uint8_t *> tab(6 * (size_t)E, nullptr);
    for (size_t u = 0; u < uniq.size(); u++) {
        const int e = uniq[u];
        const auto &src = srcs[u];
        uint64_t fp = 0;
        for (int i = 0; i < 6; i++) fp = (fp ^ fingerprint((const uint8_t *)src[i], sz[i])) * 0x100000001b3ull;
        const uint64_t key = ((uint64_t)(uint32_t)w->layer_id << 32) | (uint32_t)e;
        auto it = g.experts.find(key);
        if (it != g.experts.end() &&
            (it->second.dim != dim || it->second.inter != inter || it->second.fp != fp)) {
            (void)hipStreamSynchronize(g.stream);
            (void)hipFree(it->second.p[0]);
            g.bytes_resident -= it->second.bytes;
            g.experts.erase(it);
            it = g.experts.end();
        }
        if (it == g.experts.end()) {
            ExpertW ew{};
            size_t tot = 0;
            for (int i = 0; i < 6; i++) tot += align256(sz[i]);
            uint8_t *base = nullptr;
            if (!ok(hipMalloc(&base, tot), "hipMalloc expert")) return 1;
            size_t off = 0;
            for (int i = 0; i < 6; i++) {
                ew.p[i] = base + off;
                off += align256(sz[i]);
            }
            /* w1, w3: [inter, dim]; w2: [dim, inter] */
            const int mo[3] = {inter, dim, inter}, mk[3] = {dim, inter, dim};
            ew.dim = dim;
            ew.inter = inter;
            ew.tiled = moe_tiled(dim, inter);
            ew.fp = fp;
            for (int m = 0; m < 3; m++) {
                if (!upload_weights(APUS_W_FP4, ew.p[2 * m], ew.p[2 * m + 1], src[2 * m],
                                    src[2 * m + 1], sz[2 * m], sz[2 * m + 1], mo[m], mk[m],
                                    ew.tiled)) {
                    (void)hipFree(base);
                    return 1;
                }
            }
            ew.bytes = tot;
            g.bytes_uploaded += tot;
            g.bytes_resident += tot;
            it = g.experts.emplace(key, ew).first;
        }
        for (int i = 0; i < 6; i++) tab[(size_t)i * E + e] = it->second.p[i];
    }
    MoeWs sizes = moe_carve(nullptr, s, topk, E, dim, inter);
    void *ws = scratch_slot(7, sizes.total);
    float *dx = (float *)scratch_slot(0, (size_t)s * dim * 4);
    int32_t *didx = (int32_t *)scratch_slot(1, (size_t)nj * 4 + (size_t)nj * 4);
    float *dwgt = (float *)((uint8_t *)didx + (size_t)nj * 4);
    float *dy = (float *)out_direct(y, (size_t)s * dim * 4);
    const bool direct = dy != nullptr;
    if (!direct) dy = (float *)scratch_slot(3, (size_t)s * dim * 4);
    if (!ws || !dx || !didx || !dy) return 1;
    MoeWs mw = moe_carve(ws, s, topk, E, dim, inter);
    if (!upload(mw.tab, tab.data(), tab.size() * sizeof(void *)) ||
        !upload(dx, x, (size_t)s * dim * 4) || !upload(didx, idx, (size_t)nj * 4) ||
        !upload(dwgt, wgt, (size_t)nj * 4))
        return 1;
    const bool etiled = moe_tiled(dim, inter);
    if (moe_pipeline(E, dim, inter, w->limit, mw.tab, dx, didx, dwgt, s, topk, dy, mw, etiled,
                     nullptr, g.stream))
        return 1;
    if ((!direct && !download(y, dy, (size_t)s * dim * 4)) || !finish()) return 1;
    return 0;
}

/* ---------------------------------------------------- device entry points */

int apus_hip_swiglu_dev(const float *g, const float *u, size_t n, float limit, float *h) {
    if (!ensure_init()) return 1;
    if (!g || !u || !h) { set_err("swiglu_dev: bad arguments"); return 1; }
    return launched(apus_launch_swiglu(g, u, n, limit, h, dev_stream()), "swiglu") ? 0 : 1;
}

int apus_hip_act_quant_dev(const float *x, int M, int K, uint8_t *codes, float *scales) {
    if (!ensure_init() || !shape_ok(M, K, 1)) return 1;
    return launched(apus_launch_act_quant(x, K, nullptr, M, K, codes, scales, dev_stream()), "act_quant") ? 0 : 1;
}

int apus_hip_fp4_gemm_dev(const uint8_t *w, const uint8_t *ws, const uint8_t *acodes,
                          const float *as, float *out, int M, int O, int K, int round_out) {
    if (!ensure_init() || !shape_ok(M, K, O)) return 1;
    return gemm_dev(APUS_W_FP4 | (round_out & APUS_HIP_W_TILED), w, ws, acodes, as, out, M, O, K,
                    round_out & 1, dev_stream());
}

int apus_hip_fp8_gemm_dev(const uint8_t *w, const uint8_t *ws, const uint8_t *acodes,
                          const float *as, float *out, int M, int O, int K, int round_out) {
    if (!ensure_init() || !shape_ok(M, K, O)) return 1;
    return gemm_dev(APUS_W_FP8 | (round_out & APUS_HIP_W_TILED), w, ws, acodes, as, out, M, O, K,
                    round_out & 1, dev_stream());
}

int apus_hip_gemm_grouped_dev(int wfmt, const ApusHipGemmEnt *ents, int n_ent,
                              const uint8_t *acodes, const float *as, int O, int K, int ldo,
                              int round_out, int max_m) {
    if (!ensure_init() || !shape_ok(1, K, O)) return 1;
    const int fmt = wfmt & ~APUS_HIP_W_TILED;
    const bool tiled = (wfmt & APUS_HIP_W_TILED) != 0;
    if (fmt != APUS_W_FP4 && fmt != APUS_W_FP8) { set_err("gemm_grouped_dev: bad format"); return 1; }
    if (tiled && ((K != 2048 && K != 4096) || O % 128)) {
        set_err("gemm_grouped_dev: tiled weights need K 2048/4096 and O %% 128 == 0");
        return 1;
    }
    static_assert(sizeof(ApusHipGemmEnt) == sizeof(ApusGemmEnt), "entry layout");
    ApusGemmArgs a{};
    a.acodes = acodes; a.ascale = as; a.ents = reinterpret_cast<const ApusGemmEnt *>(ents);
    a.O = O; a.K = K; a.ldo = ldo; a.round_out = round_out; a.max_m = max_m;
    a.wtiled = tiled ? 1 : 0;
    return launched(apus_launch_gemm(fmt, &a, n_ent, dev_stream()), "gemm_grouped_dev") ? 0 : 1;
}

static int pack_dev(int wfmt, const uint8_t *w, const uint8_t *ws, uint8_t *tw, uint8_t *tws,
                    int O, int K, int unpack) {
    if (!ensure_init()) return 1;
    if ((wfmt != APUS_W_FP4 && wfmt != APUS_W_FP8) || O <= 0 || O % 16 || K <= 0 || K % 512) {
        set_err("pack_weights: needs wfmt 0/1, O %% 16 == 0, K %% 512 == 0");
        return 1;
    }
    return launched(apus_launch_pack(wfmt, w, ws, tw, tws, O, K, unpack, dev_stream()), "pack") ? 0 : 1;
}

int apus_hip_pack_weights_dev(int wfmt, const uint8_t *w, const uint8_t *ws, uint8_t *tw,
                              uint8_t *tws, int O, int K) {
    return pack_dev(wfmt, w, ws, tw, tws, O, K, 0);
}

int apus_hip_unpack_weights_dev(int wfmt, const uint8_t *tw, const uint8_t *tws, uint8_t *w,
                                uint8_t *ws, int O, int K) {
    return pack_dev(wfmt, tw, tws, w, ws, O, K, 1);
}

size_t apus_hip_linear_workspace(int M, int K) {
    return align256((size_t)M * K) + align256((size_t)M * (K / 128) * 4);
}

static int linear_dev(int wfmt, const uint8_t *w, const uint8_t *ws, const float *x, float *out,
                      int M, int K, int O, void *workspace) {
    if (!ensure_init() || !shape_ok(M, K, O)) return 1;
    const int fmt = wfmt & ~APUS_HIP_W_TILED;
    if ((fmt != APUS_W_FP4 && fmt != APUS_W_FP8) ||
        ((wfmt & APUS_HIP_W_TILED) && !tiled_shape(O, K))) {
        set_err("linear_dev: bad format, or tiled weights with K not 1024/2048/4096/8192 or O %% 128 != 0");
        return 1;
    }
    if (!workspace) { set_err("linear_dev: workspace required"); return 1; }
    const int f = linear_fused(wfmt, w, ws, x, out, M, K, O, dev_stream());
    if (f >= 0) return f;
    uint8_t *dc = (uint8_t *)workspace;
    float *dsc = (float *)(dc + align256((size_t)M * K));
    if (!launched(apus_launch_act_quant(x, K, nullptr, M, K, dc, dsc, dev_stream()), "act_quant")) return 1;
    return gemm_dev(wfmt, w, ws, dc, dsc, out, M, O, K, 1, dev_stream());
}

int apus_hip_linear_dev(int wfmt, const uint8_t *w, const uint8_t *ws, const float *x, float *out,
                        int M, int K, int O, void *workspace) {
    return linear_dev(wfmt, w, ws, x, out, M, K, O, workspace);
}

int apus_hip_fp4_linear_dev(const uint8_t *w, const uint8_t *ws, const float *x, float *out,
                            int M, int K, int O, void *workspace) {
    return linear_dev(APUS_W_FP4, w, ws, x, out, M, K, O, workspace);
}

int apus_hip_fp8_linear_dev(const uint8_t *w, const uint8_t *ws, const float *x, float *out,
                            int M, int K, int O, void *workspace) {
    return linear_dev(APUS_W_FP8, w, ws, x, out, M, K, O, workspace);
}

/* ------------------------------------------------------------- the store */

ApusHipStore *apus_hip_store_create(int n_layers, int E, int dim, int inter, char *err,
                                    size_t errcap) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!ensure_init() || n_layers <= 0 || E <= 0 || dim % 128 || inter % 128) {
        if (g_err[0] == 0) set_err("store_create: bad arguments");
        if (err && errcap) snprintf(err, errcap, "%s", g_err);
        return nullptr;
    }
    ApusHipStore *st = new ApusHipStore();
    st->L = n_layers; st->E = E; st->dim = dim; st->inter = inter;
    st->tiled = moe_tiled(dim, inter);
    const size_t sz[6] = {(size_t)inter * dim / 2, (size_t)inter * dim / 32,
                          (size_t)dim * inter / 2, (size_t)dim * inter / 32,
                          (size_t)inter * dim / 2, (size_t)inter * dim / 32};
    st->expert_bytes = 0;
    for (int i = 0; i < 6; i++) { st->sz[i] = sz[i]; st->expert_bytes += align256(sz[i]); }
    /* a failed layer frees every layer so far, its own included */
    auto fail = [&](uint8_t *base, uint8_t **tab) -> ApusHipStore * {
        if (err && errcap) snprintf(err, errcap, "%s", g_err);
        if (base) (void)hipFree(base);
        if (tab) (void)hipFree(tab);
        for (size_t i = 0; i < st->layer_base.size(); i++) {
            (void)hipFree(st->layer_base[i]);
            (void)hipFree(st->layer_tab[i]);
        }
        delete st;
        return nullptr;
    };
    for (int l = 0; l < n_layers; l++) {
        uint8_t *base = nullptr;
        uint8_t **tab = nullptr;
        if (hipMalloc(&base, st->expert_bytes * E) != hipSuccess ||
            hipMalloc(&tab, 6 * (size_t)E * sizeof(void *)) != hipSuccess) {
            set_err("store_create: HBM exhausted at layer %d", l);
            return fail(base, tab);
        }
        std::vector<uint8_t *> h(6 * (size_t)E);
        for (int e = 0; e < E; e++) {
            size_t off = 0;
            for (int i = 0; i < 6; i++) {
                h[(size_t)i * E + e] = base + st->expert_bytes * e + off;
                off += align256(sz[i]);
            }
        }
        if (!ok(hipMemcpy(tab, h.data(), h.size() * sizeof(void *), hipMemcpyHostToDevice),
                "store_create: slab table upload"))
            return fail(base, tab);
        st->layer_base.push_back(base);
        st->layer_tab.push_back(tab);
    }
    g.bytes_resident += st->expert_bytes * E * n_layers;
    return st;
}

void apus_hip_store_free(ApusHipStore *st) {
    if (!st) return;
    std::lock_guard<std::mutex> lk(g_mu);
    (void)hipStreamSynchronize(g.stream);
    for (size_t i = 0; i < st->layer_base.size(); i++) {
        (void)hipFree(st->layer_base[i]);
        (void)hipFree(st->layer_tab[i]);
    }
    g.bytes_resident -= st->expert_bytes * st->E * st->L;
    delete st;
}

uint64_t apus_hip_store_bytes(const ApusHipStore *st) {
    return st ? (uint64_t)st->expert_bytes * st->E * st->L : 0;
}

int apus_hip_store_fill_random(ApusHipStore *st, uint64_t seed) {
    if (!st) return 1;
    std::lock_guard<std::mutex> lk(g_mu);
    if (!ensure_init()) return 1;
    /* one launch per layer and tensor, generated straight into the store's
     * layout (tensor i of expert e of layer l: stream ((l * E + e) * 8 + i)) */
    const int mo[3] = {st->inter, st->dim, st->inter}, mk[3] = {st->dim, st->inter, st->dim};
    size_t off[6], o = 0;
    for (int i = 0; i < 6; i++) { off[i] = o; o += align256(st->sz[i]); }
    for (int l = 0; l < st->L; l++)
        for (int i = 0; i < 6; i++) {
            const int m = i / 2;
            if (!launched(apus_launch_store_fill(st->layer_base[l] + off[i], st->expert_bytes, st->E, mo[m],
                                                 mk[m], i & 1, st->tiled ? 1 : 0, seed,
                                                 (uint64_t)l * st->E * 8 + i, g.stream),
                          "store fill"))
                return 1;
        }
    return finish() ? 0 : 1;
}

int apus_hip_store_put(ApusHipStore *st, int layer, int eid, const ApusFp4W *w1,
                       const ApusFp4W *w2, const ApusFp4W *w3) {
    if (!st || layer < 0 || layer >= st->L || eid < 0 || eid >= st->E) return 1;
    std::lock_guard<std::mutex> lk(g_mu);
    const void *src[6] = {w1->packed, w1->scales, w2->packed, w2->scales, w3->packed, w3->scales};
    for (int i = 1; i < 6; i += 2)
        if (!e8m0_ok((const uint8_t *)src[i], st->sz[i], "store_put")) return 1;
    const int mo[3] = {st->inter, st->dim, st->inter}, mk[3] = {st->dim, st->inter, st->dim};
    uint8_t *p[6];
    size_t off = 0;
    for (int i = 0; i < 6; i++) {
        p[i] = st->layer_base[layer] + st->expert_bytes * eid + off;
        off += align256(st->sz[i]);
    }
    for (int m = 0; m < 3; m++) {
        if (!upload_weights(APUS_W_FP4, p[2 * m], p[2 * m + 1], src[2 * m], src[2 * m + 1],
                            st->sz[2 * m], st->sz[2 * m + 1], mo[m], mk[m], st->tiled))
            return 1;
        g.bytes_uploaded += st->sz[2 * m] + st->sz[2 * m + 1];
    }
    return finish() ? 0 : 1;
}

/* Container slabs -> the store. io_threads readers pread whole slabs into a
 * ring of pinned host buffers; this thread uploads each filled buffer with
 * asynchronous copies (through a device staging slab and the pack kernel when
 * the store is MFMA-tiled) and hands the buffer back once its copies are done.
 * Shapes are checked against the store before anything is read. */
int apus_hip_store_load(ApusHipStore *st, const ApusHipContainer *c, int io_threads, char *err,
                        size_t errcap) {
    auto fail = [&](const char *fmt, ...) {
        char m[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(m, sizeof m, fmt, ap);
        va_end(ap);
        set_err("%s", m);
        if (err && errcap) snprintf(err, errcap, "%s", m);
        return 1;
    };
    if (!st || !c) return fail("store_load: bad arguments");
    if (c->n_layers != st->L || c->E != st->E)
        return fail("store_load: container has %d layers x %d experts, store %d x %d", c->n_layers,
                    c->E, st->L, st->E);
    const int64_t wantO[3] = {st->inter, st->dim, st->inter}, wantK[3] = {st->dim, st->inter, st->dim};
    const size_t n = c->recs.size();
    for (size_t i = 0; i < n; i++) {
        const ApusHipSlabRec &r = c->recs[i];
        for (int t = 0; t < 3; t++)
            if (r.O[t] != wantO[t] || r.K[t] != wantK[t])
                return fail("store_load: expert %zu.%zu w%d is [%lld, %lld], the store holds [%lld, %lld]",
                            i / c->E, i % c->E, t + 1, (long long)r.O[t], (long long)r.K[t],
                            (long long)wantO[t], (long long)wantK[t]);
    }
    std::lock_guard<std::mutex> lk(g_mu);
    if (!ensure_init()) return fail("%s", g_err);
    const size_t slab = c->slab_bytes;
    const int nthr = io_threads > 0 ? std::min(io_threads, 32) : 4;
    const int nbuf = std::max(4, 2 * nthr);
    std::vector<int> fds;
    for (const std::string &sh : c->shards) {
        const std::string path = c->dir + "/" + sh;
        const int fd = open(path.c_str(), O_RDONLY);
        if (fd < 0) {
            for (int f : fds) close(f);
            return fail("store_load: cannot open %s", path.c_str());
        }
        fds.push_back(fd);
    }
    std::vector<uint8_t *> hbuf(nbuf, nullptr), dbuf(nbuf, nullptr);
    std::vector<hipEvent_t> ev(nbuf, nullptr);
    bool setup = true;
    for (int b = 0; b < nbuf && setup; b++) {
        setup = ok(hipHostMalloc((void **)&hbuf[b], slab, hipHostMallocDefault), "hipHostMalloc") &&
                ok(hipEventCreateWithFlags(&ev[b], hipEventDisableTiming), "hipEventCreate") &&
                (!st->tiled || ok(hipMalloc((void **)&dbuf[b], slab), "hipMalloc staging"));
    }
    struct Done { size_t idx; int buf; bool ok; };
    std::mutex mu;
    std::condition_variable cv;
    std::deque<int> free_bufs;
    std::deque<Done> ready;
    std::atomic<size_t> next{0};
    std::atomic<bool> stop{false};
    for (int b = 0; b < nbuf; b++) free_bufs.push_back(b);
    auto reader = [&]() {
        for (;;) {
            const size_t i = next.fetch_add(1);
            if (i >= n || stop) return;
            int b;
            {
                std::unique_lock<std::mutex> l(mu);
                cv.wait(l, [&] { return !free_bufs.empty() || stop; });
                if (stop) return;
                b = free_bufs.front();
                free_bufs.pop_front();
            }
            const ApusHipSlabRec &r = c->recs[i];
            size_t got = 0;
            bool good = true;
            while (got < slab) {
                const ssize_t k = pread(fds[r.shard], hbuf[b] + got, slab - got, (off_t)(r.off + got));
                if (k <= 0) { good = false; break; }
                got += (size_t)k;
            }
            {
                std::lock_guard<std::mutex> l(mu);
                ready.push_back({i, b, good});
            }
            cv.notify_all();
        }
    };
    std::vector<std::thread> threads;
    if (setup)
        for (int t = 0; t < nthr; t++) threads.emplace_back(reader);
    std::deque<int> pending;                      /* buffers whose copies are in flight */
    int rc = setup ? 0 : 1;
    size_t failed_idx = 0;
    for (size_t done = 0; rc == 0 && done < n; done++) {
        Done d;
        {
            std::unique_lock<std::mutex> l(mu);
            while (ready.empty()) {
                /* every buffer may be waiting on its copies: free the oldest */
                if (free_bufs.empty() && !pending.empty()) {
                    const int b = pending.front();
                    pending.pop_front();
                    l.unlock();
                    if (!ok(hipEventSynchronize(ev[b]), "hipEventSynchronize")) rc = 1;
                    l.lock();
                    free_bufs.push_back(b);
                    cv.notify_all();
                    if (rc) break;
                    continue;
                }
                cv.wait(l);
            }
            if (rc) break;
            d = ready.front();
            ready.pop_front();
        }
        if (!d.ok) { rc = 2; failed_idx = d.idx; break; }
        const int layer = (int)(d.idx / c->E), eid = (int)(d.idx % c->E);
        const ApusHipSlabRec &r = c->recs[d.idx];
        bool scales_ok = true;
        for (int m = 0; m < 3; m++)
            scales_ok = scales_ok && !memchr(hbuf[d.buf] + r.rel[2 * m + 1], 0xff, st->sz[2 * m + 1]);
        if (!scales_ok) {
            rc = 3;
            failed_idx = d.idx;
            std::lock_guard<std::mutex> l(mu);
            free_bufs.push_back(d.buf);
            break;
        }
        uint8_t *dst[6];
        size_t off = 0;
        for (int i = 0; i < 6; i++) {
            dst[i] = st->layer_base[layer] + st->expert_bytes * eid + off;
            off += align256(st->sz[i]);
        }
        for (int m = 0; m < 3 && rc == 0; m++) {
            const uint8_t *hw = hbuf[d.buf] + r.rel[2 * m], *hs = hbuf[d.buf] + r.rel[2 * m + 1];
            const size_t wb = st->sz[2 * m], sb = st->sz[2 * m + 1];
            if (!st->tiled) {
                if (!ok(hipMemcpyAsync(dst[2 * m], hw, wb, hipMemcpyHostToDevice, g.stream), "H2D") ||
                    !ok(hipMemcpyAsync(dst[2 * m + 1], hs, sb, hipMemcpyHostToDevice, g.stream), "H2D"))
                    rc = 1;
            } else {
                uint8_t *sw = dbuf[d.buf] + r.rel[2 * m], *ss = dbuf[d.buf] + r.rel[2 * m + 1];
                if (!ok(hipMemcpyAsync(sw, hw, wb, hipMemcpyHostToDevice, g.stream), "H2D") ||
                    !ok(hipMemcpyAsync(ss, hs, sb, hipMemcpyHostToDevice, g.stream), "H2D") ||
                    !launched(apus_launch_pack(APUS_W_FP4, sw, ss, dst[2 * m], dst[2 * m + 1],
                                               (int)r.O[m], (int)r.K[m], 0, g.stream), "pack"))
                    rc = 1;
            }
            g.bytes_uploaded += wb + sb;
        }
        if (rc == 0 && !ok(hipEventRecord(ev[d.buf], g.stream), "hipEventRecord")) rc = 1;
        {
            std::lock_guard<std::mutex> l(mu);
            pending.push_back(d.buf);
            /* hand back every buffer whose copies have finished */
            while (!pending.empty() && hipEventQuery(ev[pending.front()]) == hipSuccess) {
                free_bufs.push_back(pending.front());
                pending.pop_front();
            }
        }
        cv.notify_all();
    }
    {
        std::lock_guard<std::mutex> l(mu);
        stop = true;
    }
    cv.notify_all();
    for (auto &t : threads) t.join();
    if (!finish() && rc == 0) rc = 1;
    for (int b = 0; b < nbuf; b++) {
        if (hbuf[b]) (void)hipHostFree(hbuf[b]);
        if (dbuf[b]) (void)hipFree(dbuf[b]);
        if (ev[b]) (void)hipEventDestroy(ev[b]);
    }
    for (int f : fds) close(f);
    if (rc == 2)
        return fail("store_load: read of expert %zu.%zu failed (%s)", failed_idx / c->E,
                    failed_idx % c->E, c->shards[c->recs[failed_idx].shard].c_str());
    if (rc == 3)
        return fail("store_load: expert %zu.%zu has an E8M0 scale byte 255 (+inf in the reference, "
                    "NaN on the matrix cores)", failed_idx / c->E, failed_idx % c->E);
    if (rc) return fail("store_load: %s", g_err);
    return 0;
}

int apus_hip_store_get(const ApusHipStore *st, int layer, int eid, const uint8_t *ptrs[6]) {
    if (!st || layer < 0 || layer >= st->L || eid < 0 || eid >= st->E) return 1;
    size_t off = 0;
    for (int i = 0; i < 6; i++) {
        ptrs[i] = st->layer_base[layer] + st->expert_bytes * eid + off;
        off += align256(st->sz[i]);
    }
    return 0;
}

int apus_hip_store_tiled(const ApusHipStore *st) { return st && st->tiled ? 1 : 0; }

size_t apus_hip_moe_workspace(const ApusHipStore *st, int s, int topk) {
    if (!st) return 0;
    return moe_carve(nullptr, s, topk, st->E, st->dim, st->inter).total;
}

static int routed_dev(const ApusHipStore *st, int layer, const float *x, const int32_t *idx,
                      const float *wgt, int s, int topk, float limit, float *y, void *workspace) {
    MoeWs mw = moe_carve(workspace, s, topk, st->E, st->dim, st->inter);
    MoeSlab slab{st->layer_base[layer], st->expert_bytes, {}};
    size_t off = 0;
    for (int i = 0; i < 6; i++) { slab.off[i] = off; off += align256(st->sz[i]); }
    return moe_pipeline(st->E, st->dim, st->inter, limit, st->layer_tab[layer], x, idx, wgt, s,
                        topk, y, mw, st->tiled, &slab, dev_stream());
}

int apus_hip_moe_routed_dev(const ApusHipStore *st, int layer, const float *x, const int32_t *idx,
                            const float *wgt, int s, int topk, float limit, float *y,
                            void *workspace) {
    if (!st || layer < 0 || layer >= st->L || s <= 0 || topk <= 0 || !workspace) {
        set_err("moe_routed_dev: bad arguments");
        return 1;
    }
    return routed_dev(st, layer, x, idx, wgt, s, topk, limit, y, workspace);
}

int apus_hip_moe_routed_dense_dev(const ApusHipStore *st, int layer, const float *x,
                                  const int32_t *idx, const float *wgt, int s, int topk, float limit,
                                  float *y, void *workspace, const uint8_t *dw, const uint8_t *dws,
                                  int dense_tiled, float *dense_out) {
    if (!st || layer < 0 || layer >= st->L || s <= 0 || topk <= 0 || !workspace || !dw || !dws ||
        !dense_out || st->inter % 64) {
        set_err("moe_routed_dense_dev: bad arguments");
        return 1;
    }
    if (dense_tiled && !tiled_shape(2 * st->inter, st->dim)) {
        set_err("moe_routed_dense_dev: a tiled dense weight needs 2*inter %% 128 == 0 and K 1024..8192");
        return 1;
    }
    MoeWs mw = moe_carve(workspace, s, topk, st->E, st->dim, st->inter);
    MoeSlab slab{st->layer_base[layer], st->expert_bytes, {}};
    size_t off = 0;
    for (int i = 0; i < 6; i++) { slab.off[i] = off; off += align256(st->sz[i]); }
    DenseRider rd{dw, dws, dense_tiled ? 1 : 0, dense_out};
    return moe_pipeline(st->E, st->dim, st->inter, limit, st->layer_tab[layer], x, idx, wgt, s, topk, y,
                        mw, st->tiled, &slab, dev_stream(), nullptr, nullptr, nullptr, nullptr, nullptr,
                        &rd);
}

size_t apus_hip_moe_noalloc_max(void) { return APUS_NOALLOC_SCRATCH_BYTES; }

int apus_hip_moe_routed_dev_noalloc(const ApusHipStore *st, int layer, const float *x,
                                    const int32_t *idx, const float *wgt, int s, int topk,
                                    float limit, float *y) {
    /* set-up (streams, counters, the scratch address) happens in
     * apus_hip_enable / the store's creation: this call allocates nothing */
    if (!g.inited || !g.noalloc_scratch[0]) {
        set_err("moe_routed_dev_noalloc: call apus_hip_enable first");
        return 1;
    }
    if (!st || layer < 0 || layer >= st->L || s <= 0 || topk <= 0) {
        set_err("moe_routed_dev_noalloc: bad arguments");
        return 1;
    }
    if (g.cur_lane != 0) {
        /* the one static workspace is shared by every call on the device:
         * calls on two lanes could overlap and race on it */
        set_err("moe_routed_dev_noalloc: runs on lane 0 only (lane %d selected); its static workspace "
                "would be shared with concurrent calls", g.cur_lane);
        return 1;
    }
    const size_t need = moe_carve(nullptr, s, topk, st->E, st->dim, st->inter).total;
    if (need > APUS_NOALLOC_SCRATCH_BYTES) {
        set_err("moe_routed_dev_noalloc: %d tokens x top-%d need %zu bytes of workspace, the "
                "static scratch holds %zu (use apus_hip_moe_routed_dev with a workspace)",
                s, topk, need, (size_t)APUS_NOALLOC_SCRATCH_BYTES);
        return 1;
    }
    return routed_dev(st, layer, x, idx, wgt, s, topk, limit, y, g.noalloc_scratch[0]);
}

int apus_hip_moe_routed_h(const ApusHipStore *st, int s, int topk, const void *workspace,
                          uint8_t *codes, uint8_t *e8m0) {
    if (!ensure_init()) return 1;
    if (!st || s <= 0 || topk <= 0 || !workspace || !codes || !e8m0) {
        set_err("moe_routed_h: bad arguments");
        return 1;
    }
    MoeWs mw = moe_carve(const_cast<void *>(workspace), s, topk, st->E, st->dim, st->inter);
    const int nj = s * topk;
    /* the one-token kernels leave h by pair with E8M0 bytes; the sorted
     * pipeline by sorted position with fp32 scales */
    const bool pair = moe_pair_mode(st->dim, st->inter, s, topk);
    return launched(apus_launch_moe_h_gather(mw.hc, mw.hs, pair ? 0 : 1, pair ? nullptr : mw.pair, nj,
                                             st->inter, codes, e8m0, dev_stream()),
                    "moe_h_gather") ? 0 : 1;
}

/* --------------------------------------------------------------- helpers */

void *apus_hip_malloc(size_t bytes) {
    if (!ensure_init()) return nullptr;
    void *p = nullptr;
    if (!ok(hipMalloc(&p, bytes ? bytes : 1), "hipMalloc")) return nullptr;
    return p;
}

int apus_hip_free(void *p) { return ok(hipFree(p), "hipFree") ? 0 : 1; }

int apus_hip_h2d(void *dst, const void *src, size_t bytes) {
    if (!ensure_init()) return 1;
    return upload(dst, src, bytes) && finish() ? 0 : 1;
}

int apus_hip_d2h(void *dst, const void *src, size_t bytes) {
    if (!ensure_init()) return 1;
    return download(dst, src, bytes) && finish() ? 0 : 1;
}

int apus_hip_d2d(void *dst, const void *src, size_t bytes) {
    if (!ensure_init()) return 1;
    return ok(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, dev_stream()), "D2D") ? 0 : 1;
}

int apus_hip_memset(void *dst, int value, size_t bytes) {
    if (!ensure_init()) return 1;
    /* a memset node in a captured graph has given wrong results on replays
     * after the first on this hardware: refuse it (kernels that need zeroed
     * memory inside a graph clear it themselves) */
    if (capturing("apus_hip_memset")) return 1;
    return ok(hipMemsetAsync(dst, value, bytes, g.stream), "hipMemsetAsync") ? 0 : 1;
}

int apus_hip_fill_random(void *dst, size_t bytes, uint64_t seed, uint64_t stream_id, int kind) {
    if (!ensure_init()) return 1;
    return launched(apus_launch_fill((uint8_t *)dst, bytes, seed, stream_id, 0, kind, dev_stream()),
                    "fill") ? 0 : 1;
}

int apus_hip_synchronize(void) {
    if (!ensure_init()) return 1;
    return finish() ? 0 : 1;
}

int apus_hip_layer1(int mode, unsigned *faults) {
    if (!ensure_init()) return -1;
    if (mode < -1 || mode > 1) { set_err("layer1: mode -1, 0 or 1"); return -1; }
    if (mode >= 0 && capturing("apus_hip_layer1")) return -1;
    if (mode == 0) g.layer1 = false;
    if (mode == 1) g.layer1 = g.layer1_ok;
    if (faults) {
        if (capturing("apus_hip_layer1")) return -1;
        if (!ok(hipStreamSynchronize(g.stream), "hipStreamSynchronize")) return -1;
        (void)l1_fault_check();   /* its error is reported through *faults here */
        *faults = g.l1_faults;
        g.l1_faults = 0;
    }
    return g.layer1 ? 1 : 0;
}

int apus_hip_layer1_spin_limit(unsigned spins) {
    if (!ensure_init()) return 1;
    if (capturing("apus_hip_layer1_spin_limit")) return 1;
    g.l1_spin = spins;
    return 0;
}

int apus_hip_timer_start(void) {
    if (!ensure_init()) return 1;
    return ok(hipEventRecord(g.ev0, g.stream), "hipEventRecord") ? 0 : 1;
}

int apus_hip_stream_delay(int delay_us) {
    if (!ensure_init()) return 1;
    if (delay_us < 0 || delay_us > 1000000) { set_err("stream_delay: 0..1000000 us"); return 1; }
    if (capturing("apus_hip_stream_delay")) return 1;
    int khz = 0;
    if (!ok(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, 0), "hipDeviceGetAttribute"))
        return 1;
    if (khz <= 0) khz = 100000;
    const unsigned long long ticks = (unsigned long long)delay_us * (unsigned long long)khz / 1000ull;
    return launched(apus_launch_delay(ticks, g.stream), "delay") ? 0 : 1;
}

float apus_hip_timer_stop(void) {
    if (!ensure_init()) return -1.0f;
    if (!ok(hipEventRecord(g.ev1, g.stream), "hipEventRecord")) return -1.0f;
    if (!ok(hipEventSynchronize(g.ev1), "hipEventSynchronize")) return -1.0f;
    float ms = 0.0f;
    if (!ok(hipEventElapsedTime(&ms, g.ev0, g.ev1), "hipEventElapsedTime")) return -1.0f;
    return ms;
}

int apus_hip_lanes(int n) {
    if (!ensure_init()) return 1;
    if (n < 1 || n > 8) { set_err("lanes: 1..8"); return 1; }
    for (int i = g.nlanes; i < n; i++) {
        if (!ok(hipStreamCreateWithFlags(&g.lane[i], hipStreamNonBlocking), "hipStreamCreate") ||
            !ok(hipEventCreateWithFlags(&g.lane_ev[i], hipEventDisableTiming), "hipEventCreate") ||
            !alloc_pair_tickets(i))
            return 1;
        g.nlanes = i + 1;
    }
    return 0;
}

int apus_hip_lane(int i) {
    if (!ensure_init()) return 1;
    if (i < 0 || i >= g.nlanes) { set_err("lane %d not created", i); return 1; }
    g.cur_lane = i;
    return 0;
}

int apus_hip_fork(void) {
    if (!ensure_init()) return 1;
    if (!ok(hipEventRecord(g.lane_ev[0], g.lane[0]), "hipEventRecord")) return 1;
    for (int i = 1; i < g.nlanes; i++)
        if (!ok(hipStreamWaitEvent(g.lane[i], g.lane_ev[0], 0), "hipStreamWaitEvent")) return 1;
    return 0;
}

int apus_hip_join(void) {
    if (!ensure_init()) return 1;
    for (int i = 1; i < g.nlanes; i++) {
        if (!ok(hipEventRecord(g.lane_ev[i], g.lane[i]), "hipEventRecord") ||
            !ok(hipStreamWaitEvent(g.lane[0], g.lane_ev[i], 0), "hipStreamWaitEvent"))
            return 1;
    }
    g.cur_lane = 0;
    return 0;
}

int apus_hip_graph_begin(void) {
    if (!ensure_init()) return 1;
    if (g.graph_exec) { (void)hipGraphExecDestroy(g.graph_exec); g.graph_exec = nullptr; }
    if (g.graph) { (void)hipGraphDestroy(g.graph); g.graph = nullptr; }
    return ok(hipStreamBeginCapture(g.stream, hipStreamCaptureModeThreadLocal),
              "hipStreamBeginCapture") ? 0 : 1;
}

int apus_hip_graph_end(void) {
    if (!ensure_init()) return 1;
    if (!ok(hipStreamEndCapture(g.stream, &g.graph), "hipStreamEndCapture")) return 1;
    return ok(hipGraphInstantiate(&g.graph_exec, g.graph, nullptr, nullptr, 0),
              "hipGraphInstantiate") ? 0 : 1;
}

int apus_hip_graph_replay(int times) {
    if (!ensure_init() || !g.graph_exec) { set_err("graph_replay: no captured graph"); return 1; }
    for (int i = 0; i < times; i++)
        if (!ok(hipGraphLaunch(g.graph_exec, g.stream), "hipGraphLaunch")) return 1;
    return 0;
}

int apus_hip_device_info(char *name, size_t cap, int *cus) {
    if (!ensure_init()) return 1;
    hipDeviceProp_t prop;
    if (!ok(hipGetDeviceProperties(&prop, 0), "hipGetDeviceProperties")) return 1;
    if (name && cap) snprintf(name, cap, "%s %s", prop.name, prop.gcnArchName);
    if (cus) *cus = prop.multiProcessorCount;
    return 0;
}

/* ---- whole MoE sublayer (c/moe.h:369-595) ---- */

namespace {
struct MoeFwdWs {
    void *routed;                  /* apus_hip_moe_workspace bytes */
    float *sp, *sel, *wgt, *y, *sh, *g, *u, *hs;
    int32_t *idx;
    uint8_t *hc;
    void *lin;                     /* linear workspace for the shared expert */
    size_t total;
};

MoeFwdWs moe_fwd_carve(void *base, const ApusHipStore *st, int s, int topk) {
    MoeFwdWs w{};
    const size_t E = st->E, dim = st->dim, inter = st->inter, ss = s;
    size_t off = 0;
    auto take = [&](size_t n) { size_t o = off; off += align256(n); return o; };
    size_t o_r = take(moe_carve(nullptr, s, topk, st->E, st->dim, st->inter).total);
    size_t o_sp = take(ss * E * 4), o_sel = take(ss * E * 4);
    size_t o_idx = take(ss * topk * 4), o_wgt = take(ss * topk * 4);
    size_t o_y = take(ss * dim * 4), o_sh = take(ss * dim * 4);
    size_t o_g = take(ss * inter * 4), o_u = take(ss * inter * 4);
    size_t o_hc = take(ss * inter), o_hs = take(ss * (inter / 128) * 4);
    size_t o_lin = take(align256(ss * dim) + align256(ss * (dim / 128) * 4));
    w.total = off;
    if (base) {
        uint8_t *b = (uint8_t *)base;
        w.routed = b + o_r;
        w.sp = (float *)(b + o_sp); w.sel = (float *)(b + o_sel);
        w.idx = (int32_t *)(b + o_idx); w.wgt = (float *)(b + o_wgt);
        w.y = (float *)(b + o_y); w.sh = (float *)(b + o_sh);
        w.g = (float *)(b + o_g); w.u = (float *)(b + o_u);
        w.hc = b + o_hc; w.hs = (float *)(b + o_hs);
        w.lin = b + o_lin;
    }
    return w;
}
/* The FP8 shared expert sh = w2(swiglu(w1 x, w3 x)) with BF16-rounded
 * linears (c/moe.h:570-585). Up to 8 tokens: w1 and w3 in one few-row launch
 * (x quantised while staging), w2 with h = swiglu(g, u) computed and
 * quantised while staging. More tokens: act quant, GEMMs, swiglu_quant. */
int shared_expert(const ApusHipMoeLayer *ml, const float *x, int s, int dim, int inter,
                  bool tiled, const MoeFwdWs &w, hipStream_t st) {
    const int f8 = APUS_W_FP8 | (tiled ? APUS_HIP_W_TILED : 0);
    const bool fused = s <= 8 && (dim == 2048 || dim == 4096) && (inter == 2048 || inter == 4096);
    if (fused) {
        ApusGemmArgs a{};
        a.wtiled = tiled;
        a.ent0.w = ml->sw1; a.ent0.ws = ml->sw1s; a.ent0.out = w.g; a.ent0.M = s;
        a.ent1.w = ml->sw3; a.ent1.ws = ml->sw3s; a.ent1.out = w.u; a.ent1.M = s;
        a.O = inter; a.K = dim; a.ldo = inter; a.round_out = 1;
        a.asrc = APUS_A_F32; a.ax = x;
        if (!launched(apus_launch_gemm_few(APUS_W_FP8, &a, 2, 8, 0, st), "shared w1/w3")) return 1;
        ApusGemmArgs b{};
        b.wtiled = tiled;
        b.ent0.w = ml->sw2; b.ent0.ws = ml->sw2s; b.ent0.out = w.sh; b.ent0.M = s;
        b.O = dim; b.K = inter; b.ldo = dim; b.round_out = 1;
        b.asrc = APUS_A_SWIGLU; b.ax = w.g; b.au = w.u; b.limit = ml->limit;
        return launched(apus_launch_gemm_few(APUS_W_FP8, &b, 1, 8, 0, st), "shared w2") ? 0 : 1;
    }
    uint8_t *xc = (uint8_t *)w.lin;
    float *xs = (float *)((uint8_t *)w.lin + align256((size_t)s * dim));
    if (!launched(apus_launch_act_quant(x, dim, nullptr, s, dim, xc, xs, st), "shared act_quant") ||
        gemm_dev(f8, ml->sw1, ml->sw1s, xc, xs, w.g, s, inter, dim, 1, st) ||
        gemm_dev(f8, ml->sw3, ml->sw3s, xc, xs, w.u, s, inter, dim, 1, st) ||
        !launched(apus_launch_swiglu_quant(w.g, w.u, s, inter, ml->limit, w.hc, w.hs, st),
                  "shared swiglu"))
        return 1;
    return gemm_dev(f8, ml->sw2, ml->sw2s, w.hc, w.hs, w.sh, s, dim, inter, 1, st);
}
}  // namespace

size_t apus_hip_moe_forward_workspace(const ApusHipStore *st, int s, int topk) {
    if (!st || s <= 0 || topk <= 0) return 0;
    return moe_fwd_carve(nullptr, st, s, topk).total;
}

int apus_hip_moe_forward_dev(const ApusHipStore *st, int layer, const ApusHipMoeLayer *ml,
                             const float *x, const int64_t *ids, int s, int topk, float *out,
                             const ApusHipMoeInterm *interm, void *workspace) {
    if (!st || !ml || layer < 0 || layer >= st->L || s <= 0 || topk <= 0 || topk > 16 ||
        topk > st->E || !workspace || !ml->gate_w || (ml->hash && (!ml->tid2eid || !ids)) ||
        (!ml->hash && !ml->gate_bias) || st->dim % 256 || !ml->sw1 || !ml->sw2 || !ml->sw3) {
        set_err("moe_forward_dev: bad arguments");
        return 1;
    }
    if (!ensure_init()) return 1;
    const int E = st->E, dim = st->dim, inter = st->inter;
    hipStream_t sm = dev_stream();
    MoeFwdWs w = moe_fwd_carve(workspace, st, s, topk);
    /* shared expert (FP8; BF16-rounded linears, SwiGLU, c/moe.h:570-585) on
     * the side stream, beside the router and the routed experts: it needs
     * only x */
    const bool sh_tiled = ml->shared_tiled != 0;
    static const bool use_side = [] {
        const char *v = getenv("APUS_HIP_MOE_SIDE");
        return v ? atoi(v) != 0 : true;
    }();
    const bool fused = moe_pair_fused(dim, inter, s, topk) && dim % 128 == 0;
    const bool route_fused = moe_pair_mode(dim, inter, s, topk) && E <= 1024;
    const RouteFuse rf{ml->hash ? nullptr : w.sel, w.sp, ml->hash ? ml->tid2eid : nullptr,
                       ml->hash ? ids : nullptr, ml->route_scale, E};
    SharedFuse shf{{ml->sw1, ml->sw2, ml->sw3}, {ml->sw1s, ml->sw2s, ml->sw3s}, sh_tiled, w.sh, out};
    if (fused) {
        /* the shared expert runs inside the routed pair kernels */
    } else if (use_side) {
        if (!ok(hipEventRecord(g.side_fork, sm), "hipEventRecord") ||
            !ok(hipStreamWaitEvent(g.side, g.side_fork, 0), "hipStreamWaitEvent") ||
            shared_expert(ml, x, s, dim, inter, sh_tiled, w, g.side) ||
            !ok(hipEventRecord(g.side_done, g.side), "hipEventRecord"))
            return 1;
    } else if (shared_expert(ml, x, s, dim, inter, sh_tiled, w, sm)) {
        return 1;
    }
    /* router: scores, selection, weights */
    if (!launched(apus_launch_router(ml->gate_w, ml->hash ? nullptr : ml->gate_bias, x, s, dim, E,
                                     w.sp, ml->hash ? nullptr : w.sel, sm), "router") ||
        (!route_fused &&
         !launched(apus_launch_topk(ml->hash ? nullptr : w.sel, w.sp, s, E, topk,
                                    ml->hash ? ml->tid2eid : nullptr, ml->hash ? ids : nullptr,
                                    ml->route_scale, w.idx, w.wgt, sm), "topk")))
        return 1;
    /* routed experts; the last launch waits for the shared expert and also
     * writes out = bf16(routed + shared) (c/moe.h:588-589) */
    {
        const MoeWs mw = moe_carve(w.routed, s, topk, st->E, st->dim, st->inter);
        MoeSlab slab{st->layer_base[layer], st->expert_bytes, {}};
        size_t off = 0;
        for (int i = 0; i < 6; i++) { slab.off[i] = off; off += align256(st->sz[i]); }
        if (moe_pipeline(E, dim, inter, ml->limit, st->layer_tab[layer], x, w.idx, w.wgt, s, topk,
                         w.y, mw, st->tiled, &slab, sm, fused ? nullptr : w.sh, fused ? nullptr : out,
                         use_side && !fused ? g.side_done : nullptr, fused ? &shf : nullptr,
                         route_fused ? &rf : nullptr))
            return 1;
    }
    if (interm) {
        const struct { void *dst; const void *src; size_t n; } cp[5] = {
            {interm->router_scores, w.sp, (size_t)s * E * 4},
            {interm->router_idx, w.idx, (size_t)s * topk * 4},
            {interm->router_w, w.wgt, (size_t)s * topk * 4},
            {interm->moe_routed, w.y, (size_t)s * dim * 4},
            {interm->moe_shared, w.sh, (size_t)s * dim * 4}};
        for (const auto &c : cp)
            if (c.dst && !ok(hipMemcpyAsync(c.dst, c.src, c.n, hipMemcpyDeviceToDevice, sm), "D2D"))
                return 1;
    }
    return 0;
}

int apus_hip_check_e4m3_hw(unsigned *mismatches, unsigned *last_bad_bits) {
    if (!ensure_init()) return 1;
    unsigned *d = (unsigned *)scratch_slot(7, 2 * sizeof(unsigned));
    if (!d || !ok(hipMemsetAsync(d, 0, 2 * sizeof(unsigned), g.stream), "memset") ||
        !launched(apus_launch_e4m3_hw_check(d, d + 1, g.stream), "e4m3 check"))
        return 1;
    unsigned h[2];
    if (!download(h, d, sizeof h) || !finish()) return 1;
    if (mismatches) *mismatches = h[0];
    if (last_bad_bits) *last_bad_bits = h[1];
    return 0;
}

float apus_hip_host_bf16_round(float x) { return apus_bf16_rne(x); }
uint8_t apus_hip_host_e4m3_quant(float x) { return (uint8_t)apus_e4m3_code(x); }
float apus_hip_host_act_scale(float amax) { return apus_pow2_from_exp(apus_act_scale_exp(amax)); }

}  // extern "C"
