/* r3d_gemm.hip -- the gfx950 gemm_nt_q row entries (mxfp4a8 and fp8a8, decode band and
 * prefill tile; the bf16-in mxfp4a16 prefill row) behind radiance's kernel-row launch
 * signature
 *     int launch(const RadArgs* a, RadStream s)
 * (src/r3d_gemm_mxfp4.hip:1587-1588,1717-1718; src/r3d_gemm_fp8a8.hip:1054-1056,1108-1110).
 *
 * Each entry: kill-switch backstop (the registration gate in r3d_rows.cpp is where the
 * engine re-resolves), the shared preamble (operands, M = numel(Y)/N), the format plan,
 * the gfx950 chip gate, then one launch on the caller's stream.  No allocation, no
 * synchronisation, no host<->device traffic in any entry.
 */
#include <hip/hip_runtime.h>

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "r3d_band.h"
#include "r3d_dump.h"
#include "r3d_gemm_any.h"
#include "r3d_gemm_kernels.h"
#include "r3d_gemv_lines.h"
#include "r3d_gemv_quad.h"
#include "r3d_gemv_wide.h"
#include "r3d_plan.h"
#include "r3d_prefill.h"
#include "rad_plugin.h"

namespace r3d {

/* Chip gate, per device, answered once: the rows are gfx950 code objects only. */
bool chip_ok() {
    static int cache[64];                       /* 0 unknown, 1 yes, 2 no */
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
    if (cache[dev] == 0) {
        hipDeviceProp_t p;
        memset(&p, 0, sizeof p);
        const bool ok = hipGetDeviceProperties(&p, dev) == hipSuccess &&
                        strncmp(p.gcnArchName, "gfx950", 6) == 0;
        cache[dev] = ok ? 1 : 2;
    }
    return cache[dev] == 1;
}

/* Compute units of the current device, answered once per device. */
int cu_count() {
    static int cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cache[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        cache[dev] = n;
    }
    return cache[dev];
}

static void debug_once(const char* what, int key) {
    if (!env_debug()) return;
    static unsigned long long seen[4] = {0, 0, 0, 0};
    const int w = (key >> 6) & 3, b = key & 63;
    if (seen[w] & (1ull << b)) return;
    seen[w] |= 1ull << b;
    fprintf(stderr, "libr3d_gfx950: %s launched\n", what);
}

/* A launch that failed: report it on stderr (the caller's next arm takes the launch, as the
 * reference re-launches a failed arm on the same operands, src/r3d_gemm_mxfp4.hip:1666-1670,
 * 2118-2122).  R3D_GFX950_FAIL_ARM (a test lever) names arms -- "quad", "lines", "skinny",
 * "splitk" -- that report a failure without launching anything, so the fallbacks can be
 * exercised. */
static bool forced_fail(const char* arm) {
    static const char* e = getenv("R3D_GFX950_FAIL_ARM");
    return e && strstr(e, arm) != nullptr;
}

static int launch_failed(const char* what, hipError_t e) {
    fprintf(stderr, "libr3d_gfx950: %s launch FAILED (%s)\n", what,
            e == hipSuccess ? "forced by R3D_GFX950_FAIL_ARM" : hipGetErrorName(e));
    return RAD_E_DEVICE;
}

static int launch_quad(const GemmPlan& P, const QuadGeom& g, hipStream_t stream) {
    if (forced_fail("quad")) return launch_failed("quad decode GEMV", hipSuccess);
    const dim3 grid((unsigned)g.blocks), block((unsigned)(64 * g.wv));
    /* mxfp4 scale rows contiguous (pitch = K/32) in a 16-byte aligned plane: 1 KB staging loads */
    const int sc16 = P.enc == ENC_MXFP4A8 && P.bs_pitch == P.K / 32 &&
                     ((uintptr_t)P.BS & 15) == 0;
    if ((g.wv != 4 && g.wv != 7 && g.wv != 8) || (g.qpw == 2 && g.wv != 4) ||
        (g.wv == 7 && (g.chunks != 1 || P.xq)) || (g.chunks != 1 && g.chunks != 2 && g.chunks != 4) ||
        P.M < 1 || P.M > 4 || !quad_fits(P))
        return RAD_E_UNSUPPORTED;
    const int pk = quad_pack((int)P.M, g.chunks == 4 ? 2 : g.chunks == 2 ? 1 : 0, P.rblk == 128,
                             sc16 != 0, P.as_pitch == P.K / 128);
#define R3D_QUAD1(ENC_, MT_, Q_, D_, X_) R3D_QUADW(ENC_, MT_, Q_, D_, X_, 4)
#define R3D_QUADW(ENC_, MT_, Q_, D_, X_, W_)                                                \
    hipLaunchKernelGGL((gemv_quad_kernel<ENC_, MT_, Q_, D_, X_, W_>), grid, block,          \
                       (size_t)g.lds, stream, P.B, P.BS, P.A, P.AS, (int)P.N, (int)P.K,      \
                       (int)P.b_pitch, (int)P.bs_pitch, (int)P.a_pitch, pk, (int)P.as_pitch, \
                       P.Y, P.y_pitch)
#define R3D_QUAD(ENC_, MT_, D_)                                                              \
    if (P.xq && g.wv == 8) R3D_QUADW(ENC_, MT_, 1, D_, 1, 8);                                \
    else if (P.xq) R3D_QUAD1(ENC_, MT_, 1, D_, 1);                                           \
    else if (g.qpw == 2) R3D_QUAD1(ENC_, MT_, 2, D_, 0);                                     \
    else if (g.wv == 8) R3D_QUADW(ENC_, MT_, 1, D_, 0, 8);                                   \
    else if (g.wv == 7) R3D_QUADW(ENC_, MT_, 1, D_, 0, 7);                                   \
    else R3D_QUAD1(ENC_, MT_, 1, D_, 0)
#define R3D_QUAD_D(ENC_, MT_)                                                                \
    do {                                                                                     \
        switch (g.depth) {                                                                   \
        case 8: R3D_QUAD(ENC_, MT_, 8); break;                                               \
        case 4: R3D_QUAD(ENC_, MT_, 4); break;                                               \
        case 2: R3D_QUAD(ENC_, MT_, 2); break;                                               \
        default: R3D_QUAD(ENC_, MT_, 1); break;                                              \
        }                                                                                    \
    } while (0)
    if (P.enc == ENC_MXFP4A8) {
        if (g.mt == 1) R3D_QUAD_D(ENC_MXFP4A8, 1);
        else R3D_QUAD_D(ENC_MXFP4A8, 4);
    } else {
        if (g.mt == 1) R3D_QUAD_D(ENC_FP8A8, 1);
        else R3D_QUAD_D(ENC_FP8A8, 4);
    }
#undef R3D_QUAD_D
#undef R3D_QUAD
#undef R3D_QUAD1
#undef R3D_QUADW
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return launch_failed("quad decode GEMV", e);
    debug_once(P.enc == ENC_MXFP4A8 ? "mxfp4a8 quad decode GEMV" : "fp8a8 quad decode GEMV",
               128 + (P.enc << 4) + g.mt + 2 * P.xq);
    return RAD_OK;
}

/* passes > 1: P.M = 17..64 rows in 16-row passes side by side (grid.y), each pass exactly a
 * 16-row call's arithmetic; g is the 16-row geometry */
static int launch_lines(const GemmPlan& P, const LinesGeom& g, hipStream_t stream,
                        int passes = 1) {
    if (forced_fail(passes > 1 ? "skinny" : "lines"))
        return launch_failed(passes > 1 ? "skinny line GEMV" : "line decode GEMV", hipSuccess);
    const dim3 grid((unsigned)g.blocks, (unsigned)passes), block(256);
    const int64_t lim = (int64_t)1 << 31;
    if (P.M < 1 || P.M > 127 || (g.chunks != 1 && g.chunks != 2 && g.chunks != 4) ||
        P.a_pitch >= lim || P.as_pitch >= lim || P.b_pitch >= lim || P.bs_pitch >= lim ||
        g.wlds != lines_wlds(P.enc, g.tw, P.K, g.chunks))
        return RAD_E_UNSUPPORTED;
    const int pk = lines_pack((int)P.M, g.chunks == 4 ? 2 : g.chunks == 2 ? 1 : 0, P.rblk == 128,
                              P.as_pitch == P.K / 128);
#define R3D_LINES(ENC_, MT_, TW_, D_)                                                        \
    hipLaunchKernelGGL((gemv_lines_kernel<ENC_, MT_, TW_, D_>), grid, block, (size_t)g.lds,    \
                       stream, P.A, P.AS, P.B, P.BS, (int)P.N, (int)P.K, (int)P.b_pitch,     \
                       (int)P.bs_pitch, (int)P.a_pitch, pk, (int)P.as_pitch, P.Y, P.y_pitch)
#define R3D_LINES_T(ENC_, MT_, D_)                                                           \
    do {                                                                                     \
        if (g.tw == 4) R3D_LINES(ENC_, MT_, 4, (D_ > 2 ? 2 : D_));                           \
        else if (g.tw == 2) R3D_LINES(ENC_, MT_, 2, D_);                                     \
        else R3D_LINES(ENC_, MT_, 1, D_);                                                    \
    } while (0)
#define R3D_LINES_D(ENC_, MT_)                                                               \
    do {                                                                                     \
        switch (g.depth) {                                                                   \
        case 4: R3D_LINES_T(ENC_, MT_, 4); break;                                            \
        case 2: R3D_LINES_T(ENC_, MT_, 2); break;                                            \
        default: R3D_LINES_T(ENC_, MT_, 1); break;                                           \
        }                                                                                    \
    } while (0)
    if (P.enc == ENC_MXFP4A8) {
        if (g.mt == 8) R3D_LINES_D(ENC_MXFP4A8, 8);
        else R3D_LINES_D(ENC_MXFP4A8, 16);
    } else {
        if (g.mt == 8) R3D_LINES_D(ENC_FP8A8, 8);
        else R3D_LINES_D(ENC_FP8A8, 16);
    }
#undef R3D_LINES_T
#undef R3D_LINES_D
#undef R3D_LINES
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return launch_failed("line decode GEMV", e);
    debug_once(P.enc == ENC_MXFP4A8 ? "mxfp4a8 line decode GEMV" : "fp8a8 line decode GEMV",
               192 + (P.enc << 4) + g.mt);
    return RAD_OK;
}

/* The skinny-band GEMV of a K split (gemv_wide_kernel): geometry w, kc chunks of w.cg
 * groups, f32 partial planes at part. */
static hipError_t wide_launch(const GemmPlan& P, const WideGeom& w, int kc, float* part,
                              hipStream_t stream) {
    /* 32-bit lane offsets: a wave's 32 weight rows and the staged activation rows */
    const int64_t lim = (int64_t)1 << 31;
    if (32 * P.b_pitch >= lim || P.a_pitch >= lim || P.as_pitch >= lim || P.bs_pitch >= lim ||
        w.tw != 2 || P.M < 1 || P.M > 64 || w.cg < 1 || w.cg > 0xFFFF || kc < 1 || kc > 0x7FFF ||
        w.ntiles != (P.N + 255) / 256 || w.sclds != (16 * 2 * w.cg * 4 + 255) / 256 * 256)
        return hipErrorInvalidValue;
    const int pk = wide_pack((int)P.M, P.rblk == 128, P.a_pitch == P.K, P.as_pitch == P.K / 128);
    const int cgkc = w.cg | (kc << 16);
    const dim3 grid((unsigned)(w.ntiles * kc)), block(512);
#define R3D_WIDE(ENC_, D_, NTG_)                                                           \
    hipLaunchKernelGGL((gemv_wide_kernel<ENC_, 2, D_, NTG_>), grid, block, (size_t)w.lds,    \
                       stream, P.A, P.AS, P.B, P.BS, (int)P.N, (int)P.K, (int)P.b_pitch,     \
                       (int)P.bs_pitch, pk, cgkc, (int)P.a_pitch, (int)P.as_pitch, part)
#define R3D_WIDE_N(ENC_, D_)                                                                \
    switch (w.ntg) {                                                                        \
        case 1: R3D_WIDE(ENC_, D_, 1); break;                                               \
        case 2: R3D_WIDE(ENC_, D_, 2); break;                                               \
        case 3: R3D_WIDE(ENC_, D_, 3); break;                                               \
        default: R3D_WIDE(ENC_, D_, 4); break;                                              \
    }
    if (w.ntg < 1 || w.ntg > 4 || w.d != 1) return hipErrorInvalidValue;
    if (P.enc == ENC_MXFP4A8) {
        R3D_WIDE_N(ENC_MXFP4A8, 1)
    } else {
        R3D_WIDE_N(ENC_FP8A8, 1)
    }
#undef R3D_WIDE_N
#undef R3D_WIDE
    return hipGetLastError();
}

/* The in-order sum of kc f32 partial planes of M x N at part into bf16 Y. */
static hipError_t splitk_reduce(const GemmPlan& P, int kc, const float* part, hipStream_t stream) {
    const int64_t cpr = (P.N + 3) / 4;                   /* column quads a row */
    if (P.M < 1 || P.M > 65535 || cpr > 0x3FFFFFFF) return hipErrorInvalidValue;
    if (P.M * cpr <= 32768)
        hipLaunchKernelGGL((splitk_reduce_kernel<64, 16>), dim3((unsigned)((cpr + 63) / 64), (unsigned)P.M),
                           dim3(64), 0, stream, part, kc, (int)P.M, (int)P.N, P.Y, P.y_pitch);
    else
        hipLaunchKernelGGL((splitk_reduce_kernel<256, 4>), dim3((unsigned)((cpr + 255) / 256), (unsigned)P.M),
                           dim3(256), 0, stream, part, kc, (int)P.M, (int)P.N, P.Y, P.y_pitch);
    return hipGetLastError();
}

/* The skinny-band GEMV's K split, then the reduce; RAD_OK, or RAD_E_DEVICE (reported as
 * `what`) when a launch fails, for the caller's unsplit arms to recompute every element of
 * Y.  decode: the decode rows' split (named so in the R3D_DEBUG_GEMM line). */
static int launch_wide_split(const GemmPlan& P, const WideGeom& w, int kc, float* part,
                             hipStream_t stream, const char* what, bool decode, int key) {
    hipError_t e = hipSuccess;
    if (forced_fail("splitk")) return launch_failed(what, hipSuccess);
    if ((e = wide_launch(P, w, kc, part, stream)) != hipSuccess) return launch_failed(what, e);
    if ((e = splitk_reduce(P, kc, part, stream)) != hipSuccess)
        return launch_failed("split-K reduce", e);
    const bool f8 = P.enc == ENC_FP8A8;
    debug_once(decode ? (f8 ? "fp8a8 split-K decode GEMV" : "mxfp4a8 split-K decode GEMV")
                      : (f8 ? "fp8a8 split-K skinny GEMV" : "mxfp4a8 split-K skinny GEMV"),
               key);
    return RAD_OK;
}

/* The any-alignment GEMM (r3d_gemm_any.h) over A / AS as given: mode PF_A8 (e2m1 weights,
 * e4m3 A + f32 a_scale), PF_F8 (e4m3 weights) or PF_MX8 (e2m1 weights, mxfp8 A). */
static int launch_any(const GemmPlan& P, int mode, const uint8_t* A, const void* AS,
                      int64_t a_pitch, int64_t as_pitch, hipStream_t stream) {
    /* 32-bit lane offsets over one wave's 32 rows of every operand */
    const int64_t lim = (int64_t)1 << 31;
    const int64_t bsz = mode == PF_F8 ? 2 : 1, asz = mode == PF_MX8 ? 1 : 4;
    if (32 * P.b_pitch >= lim || 32 * a_pitch >= lim || 32 * P.bs_pitch * bsz >= lim ||
        32 * as_pitch * asz >= lim)
        return RAD_E_UNSUPPORTED;
    const int tm = P.M <= 16 ? 1 : 2;
    const int64_t gx = (P.N + 127) / 128, gy = (P.M + 16 * tm - 1) / (16 * tm);
    if (gx > 0x7FFFFFFF || gy > 65535) return RAD_E_SHAPE;
    const dim3 grid((unsigned)gx, (unsigned)gy), block(256);
#define R3D_ANY(MODE_, TM_)                                                                 \
    hipLaunchKernelGGL((gemm_any_kernel<MODE_, TM_>), grid, block, 0, stream, A, AS, P.B,      \
                       (const uint8_t*)P.BS, P.Y, (int)P.M, (int)P.N, (int)(P.K / 128),      \
                       P.rblk, a_pitch, as_pitch, P.b_pitch, P.bs_pitch, P.y_pitch)
    if (mode == PF_F8) {
        if (tm == 1) R3D_ANY(PF_F8, 1); else R3D_ANY(PF_F8, 2);
    } else if (mode == PF_MX8) {
        if (tm == 1) R3D_ANY(PF_MX8, 1); else R3D_ANY(PF_MX8, 2);
    } else {
        if (tm == 1) R3D_ANY(PF_A8, 1); else R3D_ANY(PF_A8, 2);
    }
#undef R3D_ANY
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return launch_failed("any-alignment GEMM", e);
    debug_once(mode == PF_F8 ? "fp8a8 any-alignment GEMM"
               : mode == PF_MX8 ? "mxfp4a16 any-alignment GEMM" : "mxfp4a8 any-alignment GEMM",
               120 + 2 * mode + (tm - 1));
    return RAD_OK;
}

/* The decode arms in order of preference -- quad GEMV (M <= 4), line GEMV (M = 5..16),
 * 16-row GEMV (any M <= 16) -- each taking the launch when the one before does not serve
 * the shape or fails to launch (a failed arm wrote nothing: the next one writes all of Y). */
static int launch_decode(const GemmPlan& P, int64_t splitk, hipStream_t stream,
                         uint8_t* part = nullptr, int64_t part_bytes = 0) {
    if (P.ua & UA_GEMM)
        return launch_any(P, P.enc == ENC_FP8A8 ? PF_F8 : PF_A8, P.A, P.AS, P.a_pitch,
                          P.as_pitch, stream);
    QuadGeom qg{};
    const bool quad = quad_fits(P) && quad_geom(P.enc, P.M, P.N, P.K, splitk, &qg, P.xq);
    /* launch scratch: the K split where it applies (decode_split_plan) */
    if (part && ((uintptr_t)part & 15) == 0 && !P.xq) {
        int kc = 0;
        WideGeom w{};
        if (decode_split_plan(P.enc, P.M, P.N, P.K, cu_count(), quad, splitk, &kc, &w) &&
            part_bytes >= (int64_t)kc * P.M * P.N * 4 &&
            launch_wide_split(P, w, kc, reinterpret_cast<float*>(part), stream,
                              "split-K decode", true, 240 + P.enc) == RAD_OK)
            return RAD_OK;
        /* no split, or a failed one: the decode arms below */
    }
    if (quad) {
        const int rc = launch_quad(P, qg, stream);
        if (rc == RAD_OK || P.xq) return rc;   /* fused bf16 activations: the quad GEMV only */
    } else if (P.xq) {
        return RAD_E_UNSUPPORTED;
    }
    LinesGeom lg{};
    if (lines_fits(P) && lines_geom(P.enc, P.M, P.N, P.K, splitk, &lg)) {
        if (launch_lines(P, lg, stream) == RAD_OK) return RAD_OK;
    }
    DecodeGeom g{};
    decode_geom(P.M, P.N, P.K, splitk, &g, gemv_wave_lds(P.enc, P.M <= 1 ? 1 : P.M <= 4 ? 4 : 16));
    const dim3 grid((unsigned)g.blocks), block((unsigned)(64 * g.waves));
    const size_t lds = (size_t)g.waves * gemv_wave_lds(P.enc, g.mt);
#define R3D_GEMV(ENC_, MT_)                                                               \
    hipLaunchKernelGGL((gemv_kernel<ENC_, MT_>), grid, block, lds, stream, P.A, P.AS, P.B,  \
                       P.BS, P.Y, (int)P.M, (int)P.N, g.steps, g.chunks, P.rblk,          \
                       P.a_pitch, P.as_pitch, P.b_pitch, P.bs_pitch, P.y_pitch)
    if (P.enc == ENC_MXFP4A8) {
        if (g.mt == 1) R3D_GEMV(ENC_MXFP4A8, 1);
        else if (g.mt == 4) R3D_GEMV(ENC_MXFP4A8, 4);
        else R3D_GEMV(ENC_MXFP4A8, 16);
    } else {
        if (g.mt == 1) R3D_GEMV(ENC_FP8A8, 1);
        else if (g.mt == 4) R3D_GEMV(ENC_FP8A8, 4);
        else R3D_GEMV(ENC_FP8A8, 16);
    }
#undef R3D_GEMV
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return launch_failed("decode GEMV", e);
    debug_once(P.enc == ENC_MXFP4A8 ? "mxfp4a8 decode GEMV" : "fp8a8 decode GEMV",
               (P.enc << 4) | (g.mt << 1));
    return RAD_OK;
}

/* The prefill GEMM: mode PF_A8 reads A/AS as given (e4m3 + f32 per 128) against e2m1
 * weights, PF_F8 the same activations against e4m3 weights with bf16 row scales, PF_MX8 the
 * mxfp8 planes the quantiser left in P.scratch.  stage (mxfp4a16 only): 0 both launches, 1
 * the quantiser alone, 2 the GEMM alone on the planes already in the scratch.  part /
 * part_bytes: launch scratch for split K's partial planes (tile_splitk); the split runs
 * when it applies and they hold tile_splitk_bytes at a 16-byte aligned address, else (and
 * when a split launch fails) the unsplit arms below take the launch. */
static int launch_prefill(const GemmPlan& P, hipStream_t stream, int stage = 0,
                          uint8_t* part = nullptr, int64_t part_bytes = 0) {
    const int mode = P.enc == ENC_MXFP4A16 ? PF_MX8 : P.enc == ENC_FP8A8 ? PF_F8 : PF_A8;
    PrefillGeom g{};
    prefill_geom(P.M, P.N, P.K, mode, cu_count(), &g);
    if (g.tiles > 0x7FFFFFFF || g.grid_m > 0x7FFFFFFF) return RAD_E_SHAPE;
    if ((P.ua & UA_GEMM) && mode != PF_MX8)
        return launch_any(P, mode, P.A, P.AS, P.a_pitch, P.as_pitch, stream);
    int cst = 0;
    PrefillGeom gs{};                                    /* the split's tile (kind 2) */
    WideGeom gw{};                                       /* or its GEMV (kind 1) */
    int kc = 0;
    const int kind = part && ((uintptr_t)part & 15) == 0 && !P.ua
                         ? splitk_plan(P.enc, P.M, P.N, P.K, cu_count(), &kc, &cst, &gs, &gw)
                         : 0;
    const bool split = kind != 0 && part_bytes >= (int64_t)kc * P.M * P.N * 4 &&
                       (kind == 1 || (gs.grid_m == 1 && gs.tiles * kc <= 0x7FFFFFFF));
    /* the skinny band on a narrow N: 16-row passes of the decode GEMVs (each output row is
     * the same arithmetic either way) */
    if (const int passes = split || P.ua ? 0 : skinny_passes(P.enc, P.M, P.N, cu_count())) {
        GemmPlan S = P;
        S.M = 16;
        LinesGeom lg{};
        int rc = RAD_E_DEVICE;
        if (lines_fits(S) && lines_geom(P.enc, 16, P.N, P.K, 0, &lg) && lg.mt == 16) {
            rc = launch_lines(P, lg, stream, passes);       /* all passes in one launch */
        } else {
            rc = RAD_OK;
            for (int p = 0; p < passes && rc == RAD_OK; ++p) {
                GemmPlan S = P;
                const int64_t m0 = 16 * (int64_t)p;
                S.M = P.M - m0 < 16 ? P.M - m0 : 16;
                S.A = P.A + m0 * P.a_pitch;
                S.AS = P.AS + m0 * P.as_pitch;
                S.Y = P.Y + m0 * P.y_pitch;
                rc = launch_decode(S, 0, stream);
            }
        }
        if (rc == RAD_OK) return RAD_OK;
        /* a failed pass: the prefill pipeline below recomputes every row of Y */
    }
    const uint8_t* A = P.A;
    const void* AS = P.AS;
    int64_t a_pitch = P.a_pitch, as_pitch = P.as_pitch;
    if (mode == PF_MX8) {
        const int64_t qbytes = ((P.M * P.K + 255) / 256) * 256;
        uint8_t* Q = P.scratch;
        uint8_t* SX = P.scratch + qbytes;
        const int64_t qblocks = P.M;                     /* one workgroup per row */
        if (qblocks > 0x7FFFFFFF) return RAD_E_SHAPE;
        if (stage != 2) {
            if (P.ua & UA_QUANT)
                hipLaunchKernelGGL(quant_mx8_kernel<true>, dim3((unsigned)qblocks), dim3(256), 0,
                                   stream, reinterpret_cast<const uint16_t*>(P.A), P.a_pitch, Q,
                                   P.K, SX, P.K / 32, P.M, (int)P.K);
            else
                hipLaunchKernelGGL(quant_mx8_kernel<false>, dim3((unsigned)qblocks), dim3(256), 0,
                                   stream, reinterpret_cast<const uint16_t*>(P.A), P.a_pitch, Q,
                                   P.K, SX, P.K / 32, P.M, (int)P.K);
        }
        if (stage == 1) {
            const hipError_t e = hipGetLastError();
            return e == hipSuccess ? RAD_OK : RAD_E_DEVICE;
        }
        A = Q;
        AS = SX;
        a_pitch = P.K;
        as_pitch = P.K / 32;
        if (P.ua & UA_GEMM) return launch_any(P, PF_MX8, A, AS, a_pitch, as_pitch, stream);
    }
    /* the kernel addresses 256 rows of any operand with 32-bit lane offsets */
    const int64_t lim = (int64_t)1 << 31;
    if (256 * a_pitch >= lim || 256 * P.b_pitch >= lim ||
        256 * (mode == PF_F8 ? 2 * P.bs_pitch : P.bs_pitch) >= lim ||
        256 * (mode == PF_MX8 ? as_pitch : 4 * as_pitch) >= lim)
        return RAD_E_UNSUPPORTED;
    /* one launch of the tile kernel of geometry g over g.tiles x ukc units (ukc = 1: the
     * whole K walk into bf16 Y; else chunks of ucst steps into the f32 planes at pp) */
    auto tiles_launch = [&](const PrefillGeom& g, int ukc, int ucst, float* pp,
                            const GemmPlan& Q) -> hipError_t {
        const dim3 grid((unsigned)(g.tiles * ukc)), block((unsigned)(64 * g.wv));
#define R3D_PF_L(MODE_, WNF_, WMF_, WV_) PrefillLayout<WNF_, WMF_, 3, MODE_ == PF_F8 ? 2 : 1, WV_>
#define R3D_PFW(MODE_, WNF_, WMF_, WV_) R3D_PFWS(MODE_, WNF_, WMF_, WV_, 0)
#define R3D_PFWS(MODE_, WNF_, WMF_, WV_, SB_)                                              \
    static_assert(R3D_PF_L(MODE_, WNF_, WMF_, WV_)::LDS ==                                 \
                      3 * prefill_stage_bytes(WNF_, WMF_, MODE_ == PF_F8 ? 2 : 1, WV_),     \
                  "host and kernel ring sizes differ");                                    \
    if ((int)R3D_PF_L(MODE_, WNF_, WMF_, WV_)::LDS != g.lds || g.wv != WV_)                 \
        return hipErrorInvalidValue;                                                        \
    hipLaunchKernelGGL((prefill_kernel<MODE_, WNF_, WMF_, WV_, SB_>), grid, block,          \
                       (size_t)(R3D_PF_L(MODE_, WNF_, WMF_, WV_)::LDS),                     \
                       stream, A, AS, Q.B, (const uint8_t*)Q.BS, Q.Y, (int)Q.M, (int)Q.N,  \
                       g.steps, (int)g.grid_m, (int)g.tiles, Q.rblk, a_pitch, as_pitch,     \
                       Q.b_pitch, Q.bs_pitch, Q.y_pitch, ukc, ucst, pp)
#define R3D_PF(MODE_, WNF_, WMF_) R3D_PFW(MODE_, WNF_, WMF_, 8)
        if (mode == PF_MX8) {
            switch (g.wnf) {
                case 8: R3D_PF(PF_MX8, 8, 4); break;
                case 7: R3D_PF(PF_MX8, 7, 4); break;
                case 6: R3D_PF(PF_MX8, 6, 4); break;
                default: R3D_PF(PF_MX8, 4, 4); break;
            }
        } else if (mode == PF_F8 && Q.rblk == 128) {
            /* the 128 x 128 block grid: one weight scale a tile and K group, folded into
             * the token's scale before the flush */
            if (g.wmf == 1) {
                R3D_PFWS(PF_F8, 4, 1, 8, 1);
            } else if (g.wv == 4) {
                R3D_PFWS(PF_F8, 4, 8, 4, 1);
            } else {
                R3D_PFWS(PF_F8, 4, 2, 8, 1);
            }
        } else if (mode == PF_F8) {
            if (g.wmf == 1) {
                R3D_PF(PF_F8, 4, 1);                    /* split K up to 64 tokens */
            } else if (g.wv == 4) {
                R3D_PFW(PF_F8, 4, 8, 4);                /* 128 x 256, one wave a SIMD */
            } else {
                R3D_PF(PF_F8, 4, 2);
            }
        } else if (g.wmf == 1) {
            R3D_PF(PF_A8, 8, 1);                        /* split K up to 64 tokens */
        } else if (g.wmf == 2) {
            R3D_PF(PF_A8, 4, 2);                        /* up to 128 tokens */
        } else {
            switch (g.wnf) {
                case 8: R3D_PF(PF_A8, 8, 4); break;
                case 7: R3D_PF(PF_A8, 7, 4); break;
                case 6: R3D_PF(PF_A8, 6, 4); break;
                default: R3D_PF(PF_A8, 4, 4); break;
            }
        }
#undef R3D_PF
#undef R3D_PFW
#undef R3D_PFWS
#undef R3D_PF_L
        return hipGetLastError();
    };
    if (split && kind == 1) {
        if (launch_wide_split(P, gw, kc, reinterpret_cast<float*>(part), stream,
                              "split-K prefill", false, 200 + 8 * mode + kind) == RAD_OK)
            return RAD_OK;
        /* a failed split: the whole K walk below recomputes every element of Y */
    } else if (split) {
        /* the prefill tile's partial planes, then their in-order sum into Y */
        hipError_t e = hipSuccess;
        if (forced_fail("splitk")) {
            launch_failed("split-K prefill", hipSuccess);
        } else if ((e = tiles_launch(gs, kc, cst, reinterpret_cast<float*>(part), P)) !=
                   hipSuccess) {
            launch_failed("split-K prefill", e);
        } else if ((e = splitk_reduce(P, kc, reinterpret_cast<const float*>(part), stream)) !=
                   hipSuccess) {
            launch_failed("split-K reduce", e);
        } else {
            debug_once(mode == PF_F8 ? "fp8a8 split-K prefill" : "mxfp4a8 split-K prefill",
                       200 + 8 * mode + kind);
            return RAD_OK;
        }
        /* a failed split: the whole K walk below recomputes every element of Y */
    }
    /* e4m3 weights on the four-wave tile: whole rounds of it over the first n1 weight rows,
     * the rest on the 128 x 128 tile (prefill_f8_split_n) */
    if (mode == PF_F8 && g.wv == 4) {
        const int64_t n1 = prefill_f8_split_n(P.M, P.N, cu_count());
        PrefillGeom g1{}, g2{};
        if (n1 > 0) {
            prefill_geom(P.M, n1, P.K, mode, cu_count(), &g1);
            prefill_geom(P.M, P.N - n1, P.K, mode, cu_count(), &g2);
        }
        if (n1 > 0 && n1 % 128 == 0 && g1.wv == 4 && g2.wv == 8) {
            GemmPlan P1 = P, P2 = P;
            P1.N = n1;
            P2.N = P.N - n1;
            P2.B = P.B + n1 * P.b_pitch;
            P2.BS = reinterpret_cast<const uint16_t*>(P.BS) + (n1 / P.rblk) * P.bs_pitch;
            P2.Y = P.Y + n1;
            hipError_t e = tiles_launch(g1, 1, g1.steps, nullptr, P1);
            if (e == hipSuccess) e = tiles_launch(g2, 1, g2.steps, nullptr, P2);
            if (e != hipSuccess) return launch_failed("prefill", e);
            debug_once("fp8a8 prefill, 128 x 256 on four waves plus a 128 x 128 remainder", 190);
            return RAD_OK;
        }
    }
    const hipError_t e = tiles_launch(g, 1, g.steps, nullptr, P);
    if (e != hipSuccess) return launch_failed("prefill", e);
    debug_once(mode == PF_MX8 ? "mxfp4a16 prefill (mxfp8 quantiser + MFMA)"
               : mode == PF_F8 ? (g.wv == 4 ? "fp8a8 prefill, 128 x 256 on four waves"
                                            : "fp8a8 prefill")
               : "mxfp4a8 prefill",
               160 + 8 * mode + g.wnf + (g.wv == 4 ? 4 : 0));
    return RAD_OK;
}

static int entry(const RadArgs* a, RadStream s, int enc, bool decode) {
    if (enc == ENC_MXFP4A16 && env_no_mxfp4()) return RAD_E_UNSUPPORTED;
    if (enc == ENC_MXFP4A8 && (env_no_mxfp4() || (decode && env_no_fp4_dec())))
        return RAD_E_UNSUPPORTED;               /* backstop: registration already hid it */
    if (enc == ENC_FP8A8 && (env_no_fp8a8() || (decode && env_no_fp8_dec())))
        return RAD_E_UNSUPPORTED;
    int64_t M = 0, N = 0;
    int rc = entry_preamble(a, enc, decode ? 16 : 0, &M, &N);
    if (rc) return rc;
    GemmPlan P{};
    rc = enc == ENC_MXFP4A8 ? plan_mxfp4a8(a, M, N, &P)
       : enc == ENC_MXFP4A16 ? plan_mxfp4a16(a, M, N, &P) : plan_fp8a8(a, M, &P);
    if (rc) return rc;
    if (!chip_ok()) return RAD_E_UNSUPPORTED;
    hipStream_t stream = (hipStream_t)s;
    if (decode)
        return launch_decode(P, decode_splitk(a), stream, (uint8_t*)a->scratch,
                             a->scratch ? a->scratch_bytes : 0);
    if (enc == ENC_MXFP4A16) return launch_prefill(P, stream);
    return launch_prefill(P, stream, 0, (uint8_t*)a->scratch, a->scratch ? a->scratch_bytes : 0);
}

/* quant_act_fp8 (src/r3d_band.hip:460-487): the reference's gates, then one wave per
 * (row, group). */
static int quant_entry(const RadArgs* a, RadStream s) {
    QuantPlan P{};
    const int rc = plan_quant_act_fp8(a, &P);
    if (rc) return rc;
    if (!chip_ok()) return RAD_E_UNSUPPORTED;
    const int64_t items = P.rows * P.ngrp;
    const int64_t blocks = (items + 3) / 4;
    if (blocks > 0x7FFFFFFF) return RAD_E_SHAPE;
    const int eb = P.x_bf16 ? 2 : 4;
    const int lanes = (int)(P.g / 8);
    const bool vec = P.g % 8 == 0 && lanes >= 1 && lanes <= 64 && (lanes & (lanes - 1)) == 0 &&
                     P.n % P.g == 0 && ((uintptr_t)P.x % 16) == 0 && (P.x_pitch * eb) % 16 == 0 &&
                     ((uintptr_t)P.q % 8) == 0 && P.q_pitch % 8 == 0;
    hipStream_t stream = (hipStream_t)s;
    if (vec) {
        /* few rows: spread each row over workgroups, one chunk a lane */
        const bool spread = P.rows <= 64;
        const dim3 sgrid((unsigned)((P.n / 8 + 255) / 256), (unsigned)P.rows);
#define R3D_QV(B_, L_)                                                                      \
    if (spread)                                                                             \
        hipLaunchKernelGGL((quant_act_fp8_spread_kernel<B_, L_>), sgrid, dim3(256), 0, stream, \
                           P.x, P.x_pitch, P.q, P.q_pitch, P.scale, P.s_pitch, P.n);          \
    else                                                                                    \
    hipLaunchKernelGGL((quant_act_fp8_vec_kernel<B_, L_>), dim3((unsigned)P.rows), dim3(256), \
                       0, stream, P.x, P.x_pitch, P.q, P.q_pitch, P.scale, P.s_pitch, P.n)
#define R3D_QVL(B_)                                                                         \
    switch (lanes) {                                                                        \
        case 1: R3D_QV(B_, 1); break;   case 2: R3D_QV(B_, 2); break;                       \
        case 4: R3D_QV(B_, 4); break;   case 8: R3D_QV(B_, 8); break;                       \
        case 16: R3D_QV(B_, 16); break; case 32: R3D_QV(B_, 32); break;                     \
        default: R3D_QV(B_, 64); break;                                                     \
    }
        if (P.x_bf16) { R3D_QVL(true); } else { R3D_QVL(false); }
#undef R3D_QVL
#undef R3D_QV
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) {
            fprintf(stderr, "libr3d_gfx950: quant_act_fp8 launch FAILED (%s)\n", hipGetErrorName(e));
            return RAD_E_DEVICE;
        }
        debug_once("quant_act_fp8 (vector)", 251);
        return RAD_OK;
    }
    const bool pair = (P.g % 2) == 0 && (P.n % 2) == 0 && (P.x_pitch % 2) == 0 &&
                      (P.q_pitch % 2) == 0 && ((uintptr_t)P.x % (2 * eb)) == 0 &&
                      ((uintptr_t)P.q % 2) == 0;
#define R3D_QA(B_, P_)                                                                      \
    hipLaunchKernelGGL((quant_act_fp8_kernel<B_, P_>), dim3((unsigned)blocks), dim3(256), 0,  \
                       stream, P.x, P.x_pitch, P.q, P.q_pitch, P.scale, P.s_pitch, P.n, P.g,  \
                       P.ngrp, items)
    if (P.x_bf16) {
        if (pair) R3D_QA(true, true); else R3D_QA(true, false);
    } else {
        if (pair) R3D_QA(false, true); else R3D_QA(false, false);
    }
#undef R3D_QA
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        fprintf(stderr, "libr3d_gfx950: quant_act_fp8 launch FAILED (%s)\n", hipGetErrorName(e));
        return RAD_E_DEVICE;
    }
    debug_once("quant_act_fp8", 250);
    return RAD_OK;
}

/* gated_quant_fp8's kernels over a plan: the vector kernel where its gates hold, else one
 * wave per (row, group). */
static int launch_gated(const GatedPlan& P, hipStream_t stream) {
    const int eb = P.gu_bf16 ? 2 : 4, ob_eb = P.ob_bf16 ? 2 : 4;
    const int lanes = (int)(P.g / 8);
    const bool vec = P.g % 8 == 0 && lanes >= 1 && lanes <= 64 && (lanes & (lanes - 1)) == 0 &&
                     P.n % P.g == 0 && ((uintptr_t)P.gu % 16) == 0 &&
                     (P.gu_pitch * eb) % 16 == 0 && ((uintptr_t)P.q % 8) == 0 &&
                     P.q_pitch % 8 == 0 &&
                     (!P.ob || (((uintptr_t)P.ob % 16) == 0 && (P.ob_pitch * ob_eb) % 16 == 0));
    if (vec) {
        const dim3 grid((unsigned)((P.n / 8 + 255) / 256), (unsigned)P.rows);
#define R3D_GV(B_, L_)                                                                      \
    hipLaunchKernelGGL((gated_quant_fp8_vec_kernel<B_, L_>), grid, dim3(256), 0, stream,      \
                       P.gu, P.gu_pitch, P.q, P.q_pitch, P.scale, P.s_pitch, P.ob, P.ob_bf16, \
                       P.ob_pitch, P.n, P.silu)
#define R3D_GVL(B_)                                                                         \
    switch (lanes) {                                                                        \
        case 1: R3D_GV(B_, 1); break;   case 2: R3D_GV(B_, 2); break;                       \
        case 4: R3D_GV(B_, 4); break;   case 8: R3D_GV(B_, 8); break;                       \
        case 16: R3D_GV(B_, 16); break; case 32: R3D_GV(B_, 32); break;                     \
        default: R3D_GV(B_, 64); break;                                                     \
    }
        if (P.gu_bf16) { R3D_GVL(true); } else { R3D_GVL(false); }
#undef R3D_GVL
#undef R3D_GV
    } else {
        const int64_t items = P.rows * P.ngrp;
        const int64_t blocks = (items + 3) / 4;
        if (blocks > 0x7FFFFFFF) return RAD_E_SHAPE;
#define R3D_GQ(B_)                                                                          \
    hipLaunchKernelGGL((gated_quant_fp8_kernel<B_>), dim3((unsigned)blocks), dim3(256), 0,    \
                       stream, P.gu, P.gu_pitch, P.q, P.q_pitch, P.scale, P.s_pitch, P.ob,    \
                       P.ob_bf16, P.ob_pitch, P.n, P.g, P.ngrp, items, P.silu)
        if (P.gu_bf16) R3D_GQ(true); else R3D_GQ(false);
#undef R3D_GQ
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        fprintf(stderr, "libr3d_gfx950: gated_quant_fp8 launch FAILED (%s)\n", hipGetErrorName(e));
        return RAD_E_DEVICE;
    }
    debug_once(vec ? "gated_quant_fp8 (vector)" : "gated_quant_fp8", vec ? 253 : 252);
    return RAD_OK;
}

/* rmsnorm_quant_fp8 (src/r3d_more.hip:482-539): the reference's gates, then one workgroup
 * per row with the row staged in LDS. */
static int rms_entry(const RadArgs* a, RadStream s) {
    RmsPlan P{};
    const int rc = plan_rmsnorm_quant_fp8(a, &P);
    if (rc) return rc;
    if (!chip_ok()) return RAD_E_UNSUPPORTED;
    hipStream_t stream = (hipStream_t)s;
    const size_t lds = (size_t)((P.n * 2 + 15) / 16 * 16);
    const int ob_eb = P.ob_bf16 ? 2 : 4;
    auto a16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    /* 16-byte row walks: 8-element chunks tiling every row, aligned bases and pitches */
    const bool vec = P.n % 8 == 0 && a16(P.x) && P.x_pitch % 8 == 0 &&
                     (!P.res || (a16(P.res) && P.r_pitch % 8 == 0)) && a16(P.w) &&
                     (!P.ob || (a16(P.ob) && (P.ob_pitch * ob_eb) % 16 == 0));
    /* vector quantiser: groups of 8..512 tiling the row, 8-byte code stores */
    const int lanes = (int)(P.g / 8);
    const bool vq = vec && P.g % 8 == 0 && lanes >= 1 && lanes <= 64 &&
                    (lanes & (lanes - 1)) == 0 && P.n % P.g == 0 &&
                    ((uintptr_t)P.q % 8) == 0 && P.q_pitch % 8 == 0;
#define R3D_RMS(W_, V_, L_)                                                                 \
    hipLaunchKernelGGL((rmsnorm_quant_fp8_kernel<W_, V_, L_>), dim3((unsigned)P.rows),        \
                       dim3(256), lds, stream, reinterpret_cast<const uint16_t*>(P.x),        \
                       P.x_pitch, reinterpret_cast<uint16_t*>(P.res), P.r_pitch, P.w, P.q,    \
                       P.q_pitch, P.scale, P.s_pitch, P.ob, P.ob_bf16, P.ob_pitch, (int)P.n,  \
                       (int)P.g, (int)P.ngrp, P.eps, P.wadd)
#define R3D_RMSL(W_)                                                                        \
    if (!vec) { R3D_RMS(W_, false, 0); }                                                    \
    else if (!vq) { R3D_RMS(W_, true, 0); }                                                 \
    else switch (lanes) {                                                                   \
        case 1: R3D_RMS(W_, true, 1); break;   case 2: R3D_RMS(W_, true, 2); break;         \
        case 4: R3D_RMS(W_, true, 4); break;   case 8: R3D_RMS(W_, true, 8); break;         \
        case 16: R3D_RMS(W_, true, 16); break; case 32: R3D_RMS(W_, true, 32); break;       \
        default: R3D_RMS(W_, true, 64); break;                                              \
    }
    if (P.w_bf16) { R3D_RMSL(true) } else { R3D_RMSL(false) }
#undef R3D_RMSL
#undef R3D_RMS
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        fprintf(stderr, "libr3d_gfx950: rmsnorm_quant_fp8 launch FAILED (%s)\n", hipGetErrorName(e));
        return RAD_E_DEVICE;
    }
    debug_once("rmsnorm_quant_fp8", 254);
    return RAD_OK;
}

/* gated_quant_fp8 (src/r3d_band.hip:492-541): the reference's gates, then the kernels. */
static int gated_entry(const RadArgs* a, RadStream s) {
    GatedPlan P{};
    const int rc = plan_gated_quant_fp8(a, &P);
    if (rc) return rc;
    if (!chip_ok()) return RAD_E_UNSUPPORTED;
    return launch_gated(P, (hipStream_t)s);
}

/* gemm_nt_q_gated at fp8a8 (src/r3d_gemm_fp8a8.hip:1166-1241): the fp8a8 GEMM writes the
 * [M, 2n] bf16 gate_up plane into the launch scratch -- the arm the gemm_nt_q rows would
 * run at this M (the decode GEMVs up to M = 16 while the fp8a8 decode row is registered,
 * else the prefill pipeline) -- then gated_quant_fp8's kernels close it into codes and
 * scales on the same stream: the two ops' composition, byte for byte. */
static int gemm_gated_entry(const RadArgs* a, RadStream s) {
    GemmPlan G{};
    GatedPlan E{};
    int rc = plan_gemm_gated(a, &G, &E);
    if (rc) return rc;
    if (!chip_ok()) return RAD_E_UNSUPPORTED;
    hipStream_t stream = (hipStream_t)s;
    const bool dec = G.M <= 16 && !env_no_fp8_dec();
    rc = dec ? launch_decode(G, decode_splitk(a), stream) : launch_prefill(G, stream);
    if (rc) return rc;
    return launch_gated(E, stream);
}

}  // namespace r3d

/* The row entries (each the launch pointer of the row named in its dump_wrap call, and the
 * name under which R3D_DUMP captures it). */
extern "C" {

int r3d_rad_quant_act_fp8(const RadArgs* a, RadStream s) {
    return r3d::dump_wrap("quant_act_fp8_act", a, s, r3d::quant_entry);
}
int r3d_rad_gated_quant_fp8(const RadArgs* a, RadStream s) {
    return r3d::dump_wrap("gated_quant_fp8_act", a, s, r3d::gated_entry);
}
int r3d_rad_rmsnorm_quant_fp8(const RadArgs* a, RadStream s) {
    return r3d::dump_wrap("rmsnorm_quant_fp8", a, s, r3d::rms_entry);
}
int r3d_rad_gemm_nt_q_gated_fp8(const RadArgs* a, RadStream s) {
    return r3d::dump_wrap("gemm_nt_q_gated_fp8a8", a, s, r3d::gemm_gated_entry);
}
int64_t r3d_rad_gemm_nt_q_gated_fp8_scratch(const RadArgs* a) {
    return r3d::gemm_gated_scratch_bytes(a);
}

int r3d_rad_gemm_nt_q(const RadArgs* a, RadStream s) {
    return r3d::dump_wrap("gemm_nt_q_mxfp4", a, s, [](const RadArgs* x, RadStream t) {
        return r3d::entry(x, t, r3d::ENC_MXFP4A8, false);
    });
}
int64_t r3d_rad_gemm_nt_q_scratch(const RadArgs* a) {
    return r3d::tile_scratch_bytes(a, r3d::ENC_MXFP4A8, r3d::cu_count());
}
int r3d_rad_gemm_nt_q_mxfp4_decode(const RadArgs* a, RadStream s) {
    return r3d::dump_wrap("gemm_nt_q_mxfp4_decode", a, s, [](const RadArgs* x, RadStream t) {
        return r3d::entry(x, t, r3d::ENC_MXFP4A8, true);
    });
}
int64_t r3d_rad_gemm_nt_q_mxfp4_decode_scratch(const RadArgs* a) {
    return r3d::decode_scratch_bytes(a, r3d::ENC_MXFP4A8, r3d::cu_count());
}
int r3d_rad_gemm_nt_q_mxfp4a16(const RadArgs* a, RadStream s) {
    return r3d::dump_wrap("gemm_nt_q_mxfp4a16", a, s, [](const RadArgs* x, RadStream t) {
        return r3d::entry(x, t, r3d::ENC_MXFP4A16, false);
    });
}
int64_t r3d_rad_gemm_nt_q_mxfp4a16_scratch(const RadArgs* a) {
    long long M = 0, K = 0;
    if (!rad_args_geti(a, "M", &M) || !rad_args_geti(a, "K", &K)) return 0;   /* 0 = none */
    if (M <= 0 || K <= 0 || M > (1LL << 27) || K > (1LL << 27)) return 0;
    return r3d::mxfp4a16_scratch_bytes(M, K);
}
int r3d_rad_gemm_nt_q_fp8(const RadArgs* a, RadStream s) {
    return r3d::dump_wrap("gemm_nt_q_fp8a8", a, s, [](const RadArgs* x, RadStream t) {
        return r3d::entry(x, t, r3d::ENC_FP8A8, false);
    });
}
int64_t r3d_rad_gemm_nt_q_fp8_scratch(const RadArgs* a) {
    return r3d::tile_scratch_bytes(a, r3d::ENC_FP8A8, r3d::cu_count());
}
int r3d_rad_gemm_nt_q_fp8_decode(const RadArgs* a, RadStream s) {
    return r3d::dump_wrap("gemm_nt_q_fp8a8_decode", a, s, [](const RadArgs* x, RadStream t) {
        return r3d::entry(x, t, r3d::ENC_FP8A8, true);
    });
}
int64_t r3d_rad_gemm_nt_q_fp8_decode_scratch(const RadArgs* a) {
    return r3d::decode_scratch_bytes(a, r3d::ENC_FP8A8, r3d::cu_count());
}
int r3d_gfx950_describe(const char* row, const RadArgs* a, char* buf, int len) {
    return r3d::describe(row, a, buf, len);
}
int r3d_gfx950_mxfp4a16_stage(const RadArgs* a, RadStream s, int stage) {
    if (stage < 0 || stage > 2) return RAD_E_INVAL;
    if (r3d::env_no_mxfp4()) return RAD_E_UNSUPPORTED;
    int64_t M = 0, N = 0;
    int rc = r3d::entry_preamble(a, r3d::ENC_MXFP4A16, 0, &M, &N);
    if (rc) return rc;
    r3d::GemmPlan P{};
    rc = r3d::plan_mxfp4a16(a, M, N, &P);
    if (rc) return rc;
    if (!r3d::chip_ok()) return RAD_E_UNSUPPORTED;
    /* the skinny band's decode-GEMV passes have no quantiser stage */
    if (r3d::skinny_passes(P.enc, P.M, P.N, r3d::cu_count())) return RAD_E_UNSUPPORTED;
    return r3d::launch_prefill(P, (hipStream_t)s, stage);
}

}  /* extern "C" */
