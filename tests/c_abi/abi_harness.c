/* abi_harness.c -- a C engine-side caller of libr3d_gfx950.so, compiled against
 * include/rad_abi.h and include/r3d_gfx950.h and linked against the library itself, so the
 * header's prototypes and the binary's exports must agree at build time.  Test
 * infrastructure (it also links the CPU oracle as the checker); modelled on the
 * reference's dlopen harness (tools/probe_m4_entry.cpp:24-97): hand-built RadTensor /
 * RadParam / RadArgs, a launch through the row table, the oracle on the host.
 *
 *   abi_harness layout   JSON: sizeof / offsetof of every ABI structure (no GPU)
 *   abi_harness table    JSON: ABI version, plugin identity, schemas and rows (no GPU)
 *   abi_harness hooks    the logits row's weight-layout hooks through RadKernelInfo with a
 *                        hand-built RadEncoding: accepted and declined encodings, the
 *                        relayout against the library's join, the unrelayout round trip
 *                        (no GPU); exit 0 when every check passes
 *   abi_harness run      one mxfp4a8 decode launch (M = 3), one fp8a8 prefill launch
 *                        (M = 130) and a split-K launch on the GPU, each through
 *                        RadKernelInfo::launch and the named export, and one logits launch
 *                        over a head the relayout hook joined (n_embd 260: the dword walk),
 *                        checked against the oracle; exit 0 when all pass
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "r3d_gfx950.h"
#include "rad_abi.h"
#include "rad_planes.h"
#include "r3d_oracle.h"

#define FIELD(T, f) printf("\"%s.%s\": [%zu, %zu], ", #T, #f, offsetof(T, f), sizeof(((T*)0)->f))

static int layout(void) {
    printf("{");
    printf("\"sizeof.RadTensor\": %zu, ", sizeof(RadTensor));
    FIELD(RadTensor, data); FIELD(RadTensor, dtype); FIELD(RadTensor, rank);
    FIELD(RadTensor, shape); FIELD(RadTensor, stride);
    printf("\"sizeof.RadParam\": %zu, ", sizeof(RadParam));
    FIELD(RadParam, kind); FIELD(RadParam, key); FIELD(RadParam, ival); FIELD(RadParam, ihi);
    FIELD(RadParam, sval); FIELD(RadParam, dval);
    printf("\"sizeof.RadTunableValue\": %zu, ", sizeof(RadTunableValue));
    FIELD(RadTunableValue, name); FIELD(RadTunableValue, value);
    printf("\"sizeof.RadArgs\": %zu, ", sizeof(RadArgs));
    FIELD(RadArgs, t); FIELD(RadArgs, n_t); FIELD(RadArgs, p); FIELD(RadArgs, n_p);
    FIELD(RadArgs, tv); FIELD(RadArgs, n_tv); FIELD(RadArgs, scratch);
    FIELD(RadArgs, scratch_bytes); FIELD(RadArgs, flags);
    printf("\"sizeof.RadTunable\": %zu, ", sizeof(RadTunable));
    FIELD(RadTunable, name); FIELD(RadTunable, values); FIELD(RadTunable, n_values);
    FIELD(RadTunable, def); FIELD(RadTunable, prose);
    printf("\"sizeof.RadConstraint\": %zu, ", sizeof(RadConstraint));
    FIELD(RadConstraint, key); FIELD(RadConstraint, op); FIELD(RadConstraint, ival);
    FIELD(RadConstraint, sval);
    printf("\"sizeof.RadKernelInfo\": %zu, ", sizeof(RadKernelInfo));
    FIELD(RadKernelInfo, name); FIELD(RadKernelInfo, op); FIELD(RadKernelInfo, family);
    FIELD(RadKernelInfo, summary); FIELD(RadKernelInfo, limits); FIELD(RadKernelInfo, formats);
    FIELD(RadKernelInfo, domain); FIELD(RadKernelInfo, priority);
    FIELD(RadKernelInfo, constraints); FIELD(RadKernelInfo, n_constraints);
    FIELD(RadKernelInfo, tunables); FIELD(RadKernelInfo, n_tunables);
    FIELD(RadKernelInfo, replaces); FIELD(RadKernelInfo, init); FIELD(RadKernelInfo, fini);
    FIELD(RadKernelInfo, launch); FIELD(RadKernelInfo, scratch); FIELD(RadKernelInfo, layout);
    FIELD(RadKernelInfo, relayout); FIELD(RadKernelInfo, opd_shape);
    FIELD(RadKernelInfo, unrelayout);
    printf("\"sizeof.RadParamSpec\": %zu, ", sizeof(RadParamSpec));
    FIELD(RadParamSpec, key); FIELD(RadParamSpec, kind); FIELD(RadParamSpec, req);
    FIELD(RadParamSpec, role);
    printf("\"sizeof.RadOperandSpec\": %zu, ", sizeof(RadOperandSpec));
    FIELD(RadOperandSpec, name); FIELD(RadOperandSpec, role); FIELD(RadOperandSpec, optional);
    printf("\"sizeof.RadOpSchema\": %zu, ", sizeof(RadOpSchema));
    FIELD(RadOpSchema, op); FIELD(RadOpSchema, params); FIELD(RadOpSchema, n_params);
    FIELD(RadOpSchema, operands); FIELD(RadOpSchema, n_operands); FIELD(RadOpSchema, prose);
    printf("\"sizeof.RadEncPlane\": %zu, ", sizeof(RadEncPlane));
    FIELD(RadEncPlane, role); FIELD(RadEncPlane, kind); FIELD(RadEncPlane, dtype);
    FIELD(RadEncPlane, block);
    printf("\"sizeof.RadEncoding\": %zu, ", sizeof(RadEncoding));
    FIELD(RadEncoding, scheme); FIELD(RadEncoding, n_planes); FIELD(RadEncoding, transform);
    FIELD(RadEncoding, plane);
    printf("\"sizeof.RadLayout\": %zu, ", sizeof(RadLayout));
    FIELD(RadLayout, tag); FIELD(RadLayout, bytes);
    printf("\"sizeof.RadPlanesHeader\": %zu, ", sizeof(RadPlanesHeader));
    FIELD(RadPlanesHeader, magic); FIELD(RadPlanesHeader, n_planes);
    FIELD(RadPlanesHeader, transform); FIELD(RadPlanesHeader, bytes);
    printf("\"sizeof.RadPlanesEntry\": %zu, ", sizeof(RadPlanesEntry));
    FIELD(RadPlanesEntry, role); FIELD(RadPlanesEntry, dtype); FIELD(RadPlanesEntry, kind);
    FIELD(RadPlanesEntry, block); FIELD(RadPlanesEntry, rows); FIELD(RadPlanesEntry, cols);
    FIELD(RadPlanesEntry, row_bytes); FIELD(RadPlanesEntry, offset);
    printf("\"sizeof.RadPluginInfo\": %zu, ", sizeof(RadPluginInfo));
    FIELD(RadPluginInfo, kind); FIELD(RadPluginInfo, name); FIELD(RadPluginInfo, version);
    FIELD(RadPluginInfo, description); FIELD(RadPluginInfo, targets);
    printf("\"RAD_MAX_RANK\": %d}\n", RAD_MAX_RANK);
    return 0;
}

/* Every declared export, referenced by name: the link fails if the binary lacks one. */
static const void* const kExports[] = {
    (const void*)rad_plugin_abi_version, (const void*)rad_plugin_info,
    (const void*)rad_kernel_schema_count, (const void*)rad_kernel_schema_at,
    (const void*)rad_kernel_count, (const void*)rad_kernel_at,
    (const void*)r3d_rad_gemm_nt_q, (const void*)r3d_rad_gemm_nt_q_mxfp4_decode,
    (const void*)r3d_rad_gemm_nt_q_fp8, (const void*)r3d_rad_gemm_nt_q_fp8_decode,
    (const void*)r3d_rad_gemm_nt_q_mxfp4a16, (const void*)r3d_rad_gemm_nt_q_mxfp4a16_scratch,
    (const void*)r3d_rad_gemm_nt_q_mxfp4a16_noalloc,
    (const void*)r3d_rad_quant_act_fp8, (const void*)r3d_rad_gated_quant_fp8,
    (const void*)r3d_rad_rmsnorm_quant_fp8, (const void*)r3d_rad_gemm_nt_q_gated_fp8,
    (const void*)r3d_rad_gemm_nt_q_gated_fp8_scratch, (const void*)r3d_gfx950_describe,
    (const void*)r3d_gfx950_mxfp4a16_stage, (const void*)r3d_gfx950_build_id,
    (const void*)r3d_rad_gemm_nt_q_scratch, (const void*)r3d_rad_gemm_nt_q_fp8_scratch,
    (const void*)r3d_rad_gemm_nt_q_mxfp4_decode_scratch,
    (const void*)r3d_rad_gemm_nt_q_fp8_decode_scratch, (const void*)r3d_rad_logits_gemm_e4m3, (const void*)r3d_gfx950_logits_head_bytes,
    (const void*)r3d_gfx950_logits_head_header, (const void*)r3d_gfx950_logits_head_join,
    (const void*)r3d_gfx950_logits_head_split, (const void*)r3d_gfx950_logits_head_forget,
    (const void*)r3d_layout_head, (const void*)r3d_relayout_head, (const void*)r3d_unrelayout_head,
    (const void*)r3d_gfx950_stream_probe,
};

static int table(void) {
    const RadPluginInfo* pi = rad_plugin_info();
    printf("{\"abi\": %u, \"exports\": %zu, \"build_id\": \"%s\", ", rad_plugin_abi_version(),
           sizeof kExports / sizeof kExports[0], r3d_gfx950_build_id());
    printf("\"plugin\": [%d, \"%s\", \"%s\"], \"schemas\": [", pi->kind, pi->name, pi->targets);
    for (int i = 0; i < rad_kernel_schema_count(); ++i) {
        const RadOpSchema* s = rad_kernel_schema_at(i);
        printf("%s[\"%s\", %d, %d]", i ? ", " : "", s->op, s->n_params, s->n_operands);
    }
    printf("], \"rows\": [");
    for (int i = 0; i < rad_kernel_count(); ++i) {
        const RadKernelInfo* k = rad_kernel_at(i);
        printf("%s[\"%s\", \"%s\", %d, %d, %d]", i ? ", " : "", k->name, k->op, k->priority,
               k->n_constraints, k->launch != NULL);
    }
    printf("]}\n");
    return 0;
}

/* ------------------------------------------------------------------ GPU run */
static uint32_t g_lcg = 777u;
static uint32_t rnd(void) { g_lcg = g_lcg * 1664525u + 1013904223u; return g_lcg >> 8; }
static uint8_t rnd_e4m3(void) {                 /* NaN-free e4m3 code */
    uint8_t c = (uint8_t)rnd();
    return (c & 0x7F) == 0x7F ? (uint8_t)(c & 0xFE) : c;
}
static float bf16f(uint16_t h) { uint32_t u = (uint32_t)h << 16; float f; memcpy(&f, &u, 4); return f; }

#define CK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { \
    fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorName(e_)); exit(2); } } while (0)

static void* to_dev(const void* h, size_t n) {
    void* d = NULL;
    CK(hipMalloc(&d, n ? n : 1));
    CK(hipMemcpy(d, h, n, hipMemcpyHostToDevice));
    return d;
}

static RadLaunchFn row_launch(const char* name) {
    for (int i = 0; i < rad_kernel_count(); ++i)
        if (strcmp(rad_kernel_at(i)->name, name) == 0) return rad_kernel_at(i)->launch;
    return NULL;
}

static RadScratchFn row_scratch(const char* name) {
    for (int i = 0; i < rad_kernel_count(); ++i)
        if (strcmp(rad_kernel_at(i)->name, name) == 0) return rad_kernel_at(i)->scratch;
    return NULL;
}

static void tensor(RadTensor* t, void* d, uint32_t dt, int64_t r, int64_t c) {
    memset(t, 0, sizeof *t);
    t->data = d; t->dtype = dt; t->rank = 2;
    t->shape[0] = r; t->shape[1] = c; t->stride[0] = c; t->stride[1] = 1;
}

/* Y from the table's launch and from the export must be equal and within the per-element
 * bound ulp_bf16 + 2K 2^-24 S + 2^-10 S8 of the oracle. */
static int check(const char* what, int64_t M, int64_t N, int64_t K, const uint16_t* Y1,
                 const uint16_t* Y2, const uint16_t* Yr, const float* Yf, const float* S,
                 const float* S8) {
    double worst = 0.0;
    int64_t bad = 0, diff = 0;
    for (int64_t i = 0; i < M * N; ++i) {
        if (Y1[i] != Y2[i]) ++diff;
        const double y = bf16f(Y1[i]), r = bf16f(Yr[i]);
        if (Y1[i] == 0xEEEE || isnan(y) != isnan(r)) { ++bad; continue; }
        if (isnan(r)) continue;
        double big = fmax(fabs(y), fabs((double)Yf[i]));
        if (big < ldexp(1.0, -126)) big = ldexp(1.0, -126);
        const double ulp = ldexp(1.0, (int)floor(log2(big)) - 7);
        const double bound = ulp + 2.0 * K * ldexp(1.0, -24) * S[i] + ldexp(1.0, -10) * S8[i];
        const double v = fabs(y - r) / bound;
        if (v > worst) worst = v;
        if (v > 1.0) ++bad;
    }
    printf("%s M=%lld N=%lld K=%lld: max_viol %.3f, outside %lld, table-vs-export differ %lld\n",
           what, (long long)M, (long long)N, (long long)K, worst, (long long)bad, (long long)diff);
    return bad == 0 && diff == 0;
}

static int run_decode_mxfp4(void) {
    const int64_t M = 3, N = 200, K = 512, asc = K / 128, bsc = K / 32;
    uint8_t* A = malloc(M * K); float* AS = malloc(M * asc * 4);
    uint8_t* B = malloc(N * K / 2); uint8_t* BS = malloc(N * bsc);
    for (int64_t i = 0; i < M * K; ++i) A[i] = rnd_e4m3();
    for (int64_t i = 0; i < M * asc; ++i) AS[i] = 0.001f + 0.01f * (float)(rnd() % 1000) / 1000.f;
    for (int64_t i = 0; i < N * K / 2; ++i) B[i] = (uint8_t)rnd();
    for (int64_t i = 0; i < N * bsc; ++i) BS[i] = (uint8_t)(115 + rnd() % 25);
    void *dA = to_dev(A, M * K), *dAS = to_dev(AS, M * asc * 4), *dB = to_dev(B, N * K / 2),
         *dBS = to_dev(BS, N * bsc), *dY1 = NULL, *dY2 = NULL;
    CK(hipMalloc(&dY1, M * N * 2)); CK(hipMalloc(&dY2, M * N * 2));
    CK(hipMemset(dY1, 0xEE, M * N * 2)); CK(hipMemset(dY2, 0xEE, M * N * 2));
    RadTensor t[7];
    tensor(&t[0], dA, RAD_F8E4M3, M, K);
    tensor(&t[1], dAS, RAD_F32, M, asc);
    tensor(&t[2], dB, RAD_FP4E2M1, N, K);                 /* FP4: strides in nibbles */
    tensor(&t[3], dBS, RAD_E8M0, N, bsc);
    tensor(&t[4], dY1, RAD_BF16, M, N);
    memset(&t[5], 0, sizeof t[5]); memset(&t[6], 0, sizeof t[6]);     /* a_sum, b_ref absent */
    const RadParam p[] = { RAD_STR("dtype", "mxfp4a8"), RAD_INT("N", N), RAD_INT("K", K),
                           RAD_INT("group", 32), RAD_INT("M", M) };
    RadArgs args = { t, 7, p, (int)(sizeof p / sizeof p[0]), NULL, 0, NULL, 0, 0 };
    char desc[512];
    r3d_gfx950_describe("gemm_nt_q_mxfp4_decode", &args, desc, sizeof desc);
    printf("decode plan: %s\n", desc);
    RadLaunchFn f = row_launch("gemm_nt_q_mxfp4_decode");
    const int rc1 = f ? f(&args, NULL) : -1;
    t[4].data = dY2;
    const int rc2 = r3d_rad_gemm_nt_q_mxfp4_decode(&args, NULL);
    CK(hipDeviceSynchronize());
    uint16_t *Y1 = malloc(M * N * 2), *Y2 = malloc(M * N * 2), *Yr = malloc(M * N * 2);
    float *Yf = malloc(M * N * 4), *S = malloc(M * N * 4), *S8 = malloc(M * N * 4);
    CK(hipMemcpy(Y1, dY1, M * N * 2, hipMemcpyDeviceToHost));
    CK(hipMemcpy(Y2, dY2, M * N * 2, hipMemcpyDeviceToHost));
    r3d_ref_quant_dot_mxfp4a8(A, K, AS, asc, B, BS, bsc, M, N, K, Yr, N, Yf, S, 1);
    r3d_ref_group8_mag(0, A, K, AS, asc, B, K / 2, BS, bsc, 1, M, N, K, S8, 1);
    const int ok = rc1 == RAD_OK && rc2 == RAD_OK &&
                   check("mxfp4a8 decode", M, N, K, Y1, Y2, Yr, Yf, S, S8);
    hipFree(dA); hipFree(dAS); hipFree(dB); hipFree(dBS); hipFree(dY1); hipFree(dY2);
    free(A); free(AS); free(B); free(BS); free(Y1); free(Y2); free(Yr); free(Yf); free(S); free(S8);
    return ok;
}

static int run_prefill_fp8(void) {
    const int64_t M = 130, N = 300, K = 384, asc = K / 128;
    uint8_t* A = malloc(M * K); float* AS = malloc(M * asc * 4);
    uint8_t* B = malloc(N * K); uint16_t* BS = malloc(N * asc * 2);
    for (int64_t i = 0; i < M * K; ++i) A[i] = rnd_e4m3();
    for (int64_t i = 0; i < M * asc; ++i) AS[i] = 0.001f + 0.01f * (float)(rnd() % 1000) / 1000.f;
    for (int64_t i = 0; i < N * K; ++i) B[i] = rnd_e4m3();
    for (int64_t i = 0; i < N * asc; ++i) BS[i] = (uint16_t)(0x3B00 + rnd() % 0x200);  /* bf16 ~0.002..0.008 */
    void *dA = to_dev(A, M * K), *dAS = to_dev(AS, M * asc * 4), *dB = to_dev(B, N * K),
         *dBS = to_dev(BS, N * asc * 2), *dY1 = NULL, *dY2 = NULL;
    CK(hipMalloc(&dY1, M * N * 2)); CK(hipMalloc(&dY2, M * N * 2));
    CK(hipMemset(dY1, 0xEE, M * N * 2)); CK(hipMemset(dY2, 0xEE, M * N * 2));
    RadTensor t[7];
    tensor(&t[0], dA, RAD_F8E4M3, M, K);
    tensor(&t[1], dAS, RAD_F32, M, asc);
    tensor(&t[2], dB, RAD_F8E4M3, N, K);
    tensor(&t[3], dBS, RAD_BF16, N, asc);                 /* per-row weight-scale grid */
    tensor(&t[4], dY1, RAD_BF16, M, N);
    memset(&t[5], 0, sizeof t[5]); memset(&t[6], 0, sizeof t[6]);
    const RadParam p[] = { RAD_STR("dtype", "fp8a8"), RAD_INT("N", N), RAD_INT("K", K),
                           RAD_INT("group", 128) };
    RadArgs args = { t, 7, p, (int)(sizeof p / sizeof p[0]), NULL, 0, NULL, 0, 0 };
    char desc[512];
    r3d_gfx950_describe("gemm_nt_q_fp8a8", &args, desc, sizeof desc);
    printf("prefill plan: %s\n", desc);
    RadLaunchFn f = row_launch("gemm_nt_q_fp8a8");
    const int rc1 = f ? f(&args, NULL) : -1;
    t[4].data = dY2;
    const int rc2 = r3d_rad_gemm_nt_q_fp8(&args, NULL);
    CK(hipDeviceSynchronize());
    uint16_t *Y1 = malloc(M * N * 2), *Y2 = malloc(M * N * 2), *Yr = malloc(M * N * 2);
    float *Yf = malloc(M * N * 4), *S = malloc(M * N * 4), *S8 = malloc(M * N * 4);
    CK(hipMemcpy(Y1, dY1, M * N * 2, hipMemcpyDeviceToHost));
    CK(hipMemcpy(Y2, dY2, M * N * 2, hipMemcpyDeviceToHost));
    r3d_ref_quant_dot_fp8a8(A, K, AS, asc, B, K, BS, asc, 1, M, N, K, Yr, N, Yf, S, 1);
    r3d_ref_group8_mag(1, A, K, AS, asc, B, K, BS, asc, 1, M, N, K, S8, 1);
    const int ok = rc1 == RAD_OK && rc2 == RAD_OK &&
                   check("fp8a8 prefill", M, N, K, Y1, Y2, Yr, Yf, S, S8);
    hipFree(dA); hipFree(dAS); hipFree(dB); hipFree(dBS); hipFree(dY1); hipFree(dY2);
    free(A); free(AS); free(B); free(BS); free(Y1); free(Y2); free(Yr); free(Yf); free(S); free(S8);
    return ok;
}

/* The mxfp4a8 tile row as an engine drives it: launch scratch sized by the row's own hook
 * (split K at this narrow N), the table's launch and the export on the same scratch. */
static int run_splitk_mxfp4(void) {
    const int64_t M = 40, N = 1000, K = 2048, asc = K / 128, bsc = K / 32;
    uint8_t* A = malloc(M * K); float* AS = malloc(M * asc * 4);
    uint8_t* B = malloc(N * K / 2); uint8_t* BS = malloc(N * bsc);
    for (int64_t i = 0; i < M * K; ++i) A[i] = rnd_e4m3();
    for (int64_t i = 0; i < M * asc; ++i) AS[i] = 0.001f + 0.01f * (float)(rnd() % 1000) / 1000.f;
    for (int64_t i = 0; i < N * K / 2; ++i) B[i] = (uint8_t)rnd();
    for (int64_t i = 0; i < N * bsc; ++i) BS[i] = (uint8_t)(115 + rnd() % 25);
    void *dA = to_dev(A, M * K), *dAS = to_dev(AS, M * asc * 4), *dB = to_dev(B, N * K / 2),
         *dBS = to_dev(BS, N * bsc), *dY1 = NULL, *dY2 = NULL, *dS = NULL;
    CK(hipMalloc(&dY1, M * N * 2)); CK(hipMalloc(&dY2, M * N * 2));
    CK(hipMemset(dY1, 0xEE, M * N * 2)); CK(hipMemset(dY2, 0xEE, M * N * 2));
    RadTensor t[7];
    tensor(&t[0], dA, RAD_F8E4M3, M, K);
    tensor(&t[1], dAS, RAD_F32, M, asc);
    tensor(&t[2], dB, RAD_FP4E2M1, N, K);
    tensor(&t[3], dBS, RAD_E8M0, N, bsc);
    tensor(&t[4], dY1, RAD_BF16, M, N);
    memset(&t[5], 0, sizeof t[5]); memset(&t[6], 0, sizeof t[6]);
    const RadParam p[] = { RAD_STR("dtype", "mxfp4a8"), RAD_INT("N", N), RAD_INT("K", K),
                           RAD_INT("group", 32) };
    RadArgs args = { t, 7, p, (int)(sizeof p / sizeof p[0]), NULL, 0, NULL, 0, 0 };
    RadScratchFn hook = row_scratch("gemm_nt_q_mxfp4");
    const int64_t need = hook ? hook(&args) : 0;
    if (need != r3d_rad_gemm_nt_q_scratch(&args) || need <= 0) {
        printf("split-K hook: %lld bytes\n", (long long)need);
        return 0;
    }
    CK(hipMalloc(&dS, (size_t)need));
    args.scratch = dS;
    args.scratch_bytes = need;
    char desc[512];
    r3d_gfx950_describe("gemm_nt_q_mxfp4", &args, desc, sizeof desc);
    printf("split-K plan: %s (hook %lld bytes)\n", desc, (long long)need);
    RadLaunchFn f = row_launch("gemm_nt_q_mxfp4");
    const int rc1 = f ? f(&args, NULL) : -1;
    t[4].data = dY2;
    const int rc2 = r3d_rad_gemm_nt_q(&args, NULL);
    CK(hipDeviceSynchronize());
    uint16_t *Y1 = malloc(M * N * 2), *Y2 = malloc(M * N * 2), *Yr = malloc(M * N * 2);
    float *Yf = malloc(M * N * 4), *S = malloc(M * N * 4), *S8 = malloc(M * N * 4);
    CK(hipMemcpy(Y1, dY1, M * N * 2, hipMemcpyDeviceToHost));
    CK(hipMemcpy(Y2, dY2, M * N * 2, hipMemcpyDeviceToHost));
    r3d_ref_quant_dot_mxfp4a8(A, K, AS, asc, B, BS, bsc, M, N, K, Yr, N, Yf, S, 1);
    r3d_ref_group8_mag(0, A, K, AS, asc, B, K / 2, BS, bsc, 1, M, N, K, S8, 1);
    const int ok = rc1 == RAD_OK && rc2 == RAD_OK && strstr(desc, "arm=splitk") != NULL &&
                   check("mxfp4a8 split-K tile", M, N, K, Y1, Y2, Yr, Yf, S, S8);
    hipFree(dA); hipFree(dAS); hipFree(dB); hipFree(dBS); hipFree(dY1); hipFree(dY2); hipFree(dS);
    free(A); free(AS); free(B); free(BS); free(Y1); free(Y2); free(Yr); free(Yf); free(S); free(S8);
    return ok;
}

/* ------------------------------------------------------------------ layout hooks */
static const RadKernelInfo* row_info(const char* name) {
    for (int i = 0; i < rad_kernel_count(); ++i)
        if (strcmp(rad_kernel_at(i)->name, name) == 0) return rad_kernel_at(i);
    return NULL;
}

/* The encoding an engine declares for a joined e4m3 head: "affine", codes (tiled 1 x 1
 * e4m3) and scale (tiled bf16, block br x 128). */
static void head_enc(RadEncoding* e, int64_t br) {
    memset(e, 0, sizeof *e);
    strcpy(e->scheme, "affine");
    e->n_planes = 2;
    strcpy(e->plane[0].role, "codes");
    e->plane[0].kind = RAD_PLANE_TILED; e->plane[0].dtype = RAD_F8E4M3;
    e->plane[0].block[0] = 1; e->plane[0].block[1] = 1;
    strcpy(e->plane[1].role, "scale");
    e->plane[1].kind = RAD_PLANE_TILED; e->plane[1].dtype = RAD_BF16;
    e->plane[1].block[0] = br; e->plane[1].block[1] = 128;
}

/* A synthetic N x K head: e4m3 codes (no NaN) and bf16 scales near 2^-7, per (br, 128). */
static void head_planes(int64_t N, int64_t K, int64_t br, uint8_t* codes, uint16_t* scale) {
    for (int64_t i = 0; i < N * K; ++i) codes[i] = rnd_e4m3();
    const int64_t sr = (N + br - 1) / br, sc = (K + 127) / 128;
    for (int64_t i = 0; i < sr * sc; ++i) scale[i] = (uint16_t)(0x3C00 + (rnd() & 0x7F));
}

#define HOOK_CK(cond, what) do { if (!(cond)) { \
    fprintf(stderr, "hooks: %s FAILED\n", what); ok = 0; } } while (0)

static int hooks(void) {
    int ok = 1;
    const RadKernelInfo* k = row_info("logits_gemm_e4m3");
    if (!k || !k->layout || !k->relayout || !k->unrelayout) {
        fprintf(stderr, "hooks: logits_gemm_e4m3 row or its hooks missing\n");
        return 1;
    }
    const int64_t N = 300, K = 260, br = 1, sr = N, sc = (K + 127) / 128;
    uint8_t* codes = malloc((size_t)(N * K));
    uint16_t* scale = malloc((size_t)(sr * sc * 2));
    head_planes(N, K, br, codes, scale);
    RadEncoding enc;
    head_enc(&enc, br);
    const int sel[2] = {0, 1};
    RadTensor pl[2];
    tensor(&pl[0], NULL, RAD_F8E4M3, N, K);              /* declare time: geometry only */
    tensor(&pl[1], NULL, RAD_BF16, sr, sc);
    RadParam p[2] = {RAD_INT("n_vocab", N), RAD_INT("n_embd", K)};
    RadLayout lay;
    memset(&lay, 0, sizeof lay);
    HOOK_CK(k->layout(p, 2, 1, &enc, sel, pl, 2, &lay) == RAD_OK, "layout accepts the head");
    const int64_t nb = r3d_gfx950_logits_head_bytes(N, K, RAD_BF16, br);
    HOOK_CK(lay.tag && strcmp(lay.tag, RAD_PLANES_TAG) == 0 && lay.bytes == nb, "layout tag / bytes");
    uint8_t* blob = malloc((size_t)nb);
    uint8_t* ref = malloc((size_t)nb);
    HOOK_CK(k->relayout(p, 2, 1, &enc, sel, pl, 2, blob, nb) == RAD_E_INVAL,
            "relayout refuses planes without data");
    pl[0].data = codes;
    pl[1].data = scale;
    HOOK_CK(k->relayout(p, 2, 1, &enc, sel, pl, 2, blob, nb - 1) == RAD_E_SHAPE,
            "relayout refuses a short destination");
    HOOK_CK(k->relayout(p, 2, 1, &enc, sel, pl, 2, blob, nb) == RAD_OK, "relayout");
    HOOK_CK(r3d_gfx950_logits_head_join(codes, K, scale, sc * 2, N, K, RAD_BF16, br, ref, nb) ==
                RAD_OK && memcmp(blob, ref, (size_t)nb) == 0,
            "relayout writes the library's join, byte for byte");
    uint8_t* c2 = calloc((size_t)(N * K), 1);
    uint16_t* s2 = calloc((size_t)(sr * sc), 2);
    RadTensor back[2];
    tensor(&back[0], c2, RAD_F8E4M3, N, K);
    tensor(&back[1], s2, RAD_BF16, sr, sc);
    HOOK_CK(k->unrelayout(p, 2, 1, &enc, sel, blob, nb, back, 2) == RAD_OK &&
                memcmp(c2, codes, (size_t)(N * K)) == 0 &&
                memcmp(s2, scale, (size_t)(sr * sc * 2)) == 0,
            "unrelayout round trip");
    /* declines */
    RadEncoding e2 = enc;
    strcpy(e2.scheme, "none");
    HOOK_CK(k->layout(p, 2, 1, &e2, sel, pl, 2, &lay) == RAD_E_DTYPE, "non-affine declined");
    e2 = enc;
    e2.transform[0] = 1;
    HOOK_CK(k->layout(p, 2, 1, &e2, sel, pl, 2, &lay) == RAD_E_DTYPE, "rotated declined");
    e2 = enc;
    e2.plane[0].dtype = RAD_I8;
    HOOK_CK(k->layout(p, 2, 1, &e2, sel, pl, 2, &lay) == RAD_E_DTYPE, "int8 codes declined");
    HOOK_CK(k->layout(p, 2, 1, NULL, NULL, pl, 1, &lay) == RAD_E_DTYPE, "plain head declined");
    HOOK_CK(k->layout(p, 2, 0, &enc, sel, pl, 2, &lay) == RAD_E_UNSUPPORTED,
            "another operand stored as is");
    printf("%s\n", ok ? "PASS" : "FAIL");
    free(codes); free(scale); free(blob); free(ref); free(c2); free(s2);
    return ok ? 0 : 1;
}

/* The logits row over a head the relayout hook joined, n_embd 260 (off a multiple of 16:
 * the dword walk), M = 3, checked per element against the oracle within
 * (2K + 300) 2^-24 S. */
static int run_logits_relayout(void) {
    const RadKernelInfo* k = row_info("logits_gemm_e4m3");
    const int64_t M = 3, N = 300, K = 260, br = 1, sr = N, sc = (K + 127) / 128;
    uint8_t* codes = malloc((size_t)(N * K));
    uint16_t* scale = malloc((size_t)(sr * sc * 2));
    head_planes(N, K, br, codes, scale);
    RadEncoding enc;
    head_enc(&enc, br);
    const int sel[2] = {0, 1};
    RadTensor pl[2];
    tensor(&pl[0], codes, RAD_F8E4M3, N, K);
    tensor(&pl[1], scale, RAD_BF16, sr, sc);
    RadParam p[4] = {RAD_INT("M", M), RAD_INT("n_vocab", N), RAD_INT("n_embd", K),
                     RAD_STR("dtype", "bf16")};
    RadLayout lay;
    if (!k || k->layout(p, 4, 1, &enc, sel, pl, 2, &lay) != RAD_OK) {
        fprintf(stderr, "logits relayout: layout declined\n");
        return 0;
    }
    uint8_t* blob = malloc((size_t)lay.bytes);
    if (k->relayout(p, 4, 1, &enc, sel, pl, 2, blob, lay.bytes) != RAD_OK) {
        fprintf(stderr, "logits relayout: relayout refused\n");
        return 0;
    }
    uint16_t* x = malloc((size_t)(M * K * 2));
    for (int64_t i = 0; i < M * K; ++i) x[i] = (uint16_t)(0x3E00 + (rnd() & 0x1FF)) ^ (uint16_t)((rnd() & 1) << 15);
    float* Y = malloc((size_t)(M * N * 4));
    float* Yr = malloc((size_t)(M * N * 4));
    float* S = malloc((size_t)(M * N * 4));
    void* dx = to_dev(x, (size_t)(M * K * 2));
    void* dw = to_dev(blob, (size_t)lay.bytes);
    void* dy = NULL;
    CK(hipMalloc(&dy, (size_t)(M * N * 4)));
    CK(hipMemset(dy, 0xFF, (size_t)(M * N * 4)));
    RadTensor t[3];
    tensor(&t[0], dx, RAD_BF16, M, K);
    memset(&t[1], 0, sizeof t[1]);
    t[1].data = dw; t[1].dtype = RAD_U8; t[1].rank = 1; t[1].shape[0] = lay.bytes; t[1].stride[0] = 1;
    tensor(&t[2], dy, RAD_F32, M, N);
    const RadArgs a = {t, 3, p, 4, NULL, 0, NULL, 0, 0};
    const int rc = k->launch(&a, NULL);
    CK(hipDeviceSynchronize());
    CK(hipMemcpy(Y, dy, (size_t)(M * N * 4), hipMemcpyDeviceToHost));
    r3d_ref_logits_e4m3(x, K, codes, scale, 0, sc, (int)br, M, N, K, Yr, N, S, 4);
    int bad = 0;
    for (int64_t i = 0; i < M * N; ++i) {
        const double tol = (2.0 * K + 300.0) * ldexp(1.0, -24) * S[i] + 1e-30;
        if (!(fabs((double)Y[i] - (double)Yr[i]) <= tol)) ++bad;
    }
    printf("logits over the relayout hook's blob (M=%lld N=%lld K=%lld): rc=%d, %d of %lld "
           "outside the bound\n", (long long)M, (long long)N, (long long)K, rc, bad,
           (long long)(M * N));
    r3d_gfx950_logits_head_forget(dw);
    CK(hipFree(dx)); CK(hipFree(dw)); CK(hipFree(dy));
    free(codes); free(scale); free(blob); free(x); free(Y); free(Yr); free(S);
    return rc == RAD_OK && bad == 0;
}

int main(int argc, char** argv) {
    const char* mode = argc > 1 ? argv[1] : "layout";
    if (strcmp(mode, "layout") == 0) return layout();
    if (strcmp(mode, "table") == 0) return table();
    if (strcmp(mode, "run") == 0) {
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess || n < 1) {
            fprintf(stderr, "no GPU\n");
            return 3;
        }
        const int a = run_decode_mxfp4();
        const int b = run_prefill_fp8();
        const int c = run_splitk_mxfp4();
        const int d = run_logits_relayout();
        printf("%s\n", a && b && c && d ? "PASS" : "FAIL");
        return a && b && c && d ? 0 : 1;
    }
    if (strcmp(mode, "hooks") == 0) return hooks();
    fprintf(stderr, "usage: abi_harness layout|table|hooks|run\n");
    return 2;
}
