/*
 * apus_hip_weak.c — weak fallbacks of the backend's engine-facing entry
 * points, for the apus translation unit that defines the hook table
 * (the counterpart of the weak apus_metal_* stubs in c/attn.h:205-243).
 *
 * An apus binary built without the HIP backend compiles this file in and
 * links: apus_hip_enable() then reports that the backend is absent, every
 * hook-shaped entry point returns nonzero (the caller runs its CPU kernel)
 * and the counters read zero. A binary that also links the backend's
 * objects (or libapus_hip.a) gets their strong definitions instead. Plain
 * C11, no HIP headers needed.
 */
#include <stdio.h>

#include "../../include/apus_hip.h"

#define APUS_WEAK __attribute__((weak))

APUS_WEAK int apus_hip_enable(char *err, size_t errcap) {
    if (err && errcap) snprintf(err, errcap, "hip backend not compiled in (make hip=1)");
    return -1;
}
APUS_WEAK void apus_hip_disable(void) {}
APUS_WEAK int apus_hip_is_enabled(void) { return 0; }
APUS_WEAK const ApusHipHooks *apus_hip_hooks(void) {
    static const ApusHipHooks none;        /* all NULL: CPU kernels */
    return &none;
}
APUS_WEAK uint64_t apus_hip_bytes_uploaded(void) { return 0; }
APUS_WEAK uint64_t apus_hip_bytes_resident(void) { return 0; }
APUS_WEAK uint64_t apus_hip_dispatches(void) { return 0; }

APUS_WEAK int apus_hip_fp8_linear(const ApusFp8W *w, const float *x, float *out, int M, int K,
                                  int O) {
    (void)w; (void)x; (void)out; (void)M; (void)K; (void)O;
    return 1;
}
APUS_WEAK int apus_hip_fp4_linear(const ApusFp4W *w, const float *x, float *out, int M, int K,
                                  int O) {
    (void)w; (void)x; (void)out; (void)M; (void)K; (void)O;
    return 1;
}
APUS_WEAK int apus_hip_f32_linear(const float *w, const float *x, float *out, int M, int K, int O,
                                  int flags) {
    (void)w; (void)x; (void)out; (void)M; (void)K; (void)O; (void)flags;
    return 1;
}
APUS_WEAK int apus_hip_head_gemv(const ApusStTensor *head, const float *x, float *out, int64_t O,
                                 int64_t K) {
    (void)head; (void)x; (void)out; (void)O; (void)K;
    return 1;
}
APUS_WEAK int apus_hip_fp4_gemm_grouped(const ApusFp4GemmEnt *ents, size_t n_ent,
                                        const uint8_t *acodes, const float *as, size_t O,
                                        size_t K) {
    (void)ents; (void)n_ent; (void)acodes; (void)as; (void)O; (void)K;
    return 1;
}
APUS_WEAK int apus_hip_moe_routed(const ApusMoeW *w, const float *x, const int32_t *idx,
                                  const float *wgt, int s, float *y) {
    (void)w; (void)x; (void)idx; (void)wgt; (void)s; (void)y;
    return 1;
}
APUS_WEAK int apus_hip_act_quant(const float *x, int M, int K, uint8_t *codes, float *scales) {
    (void)x; (void)M; (void)K; (void)codes; (void)scales;
    return 1;
}
APUS_WEAK int apus_hip_fp4_gemm(const uint8_t *w, const uint8_t *ws, const uint8_t *acodes,
                                const float *as, float *out, int M, int O, int K) {
    (void)w; (void)ws; (void)acodes; (void)as; (void)out; (void)M; (void)O; (void)K;
    return 1;
}
APUS_WEAK int apus_hip_fp8_gemm(const uint8_t *w, const uint8_t *ws, const uint8_t *acodes,
                                const float *as, float *out, int M, int O, int K) {
    (void)w; (void)ws; (void)acodes; (void)as; (void)out; (void)M; (void)O; (void)K;
    return 1;
}
APUS_WEAK const char *apus_hip_last_error(void) { return "hip backend not compiled in"; }
