/* r3d_plan.cpp -- host plans for the gfx950 gemm_nt_q rows (see r3d_plan.h). */
#include "r3d_plan.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "rad_planes.h"
#include "rad_plugin.h"
#include "r3d_gemv_layout.h"
#include "r3d_prefill_layout.h"

namespace r3d {

/* libref grid_block as the reference restates it (src/r3d_gemm_mxfp4.hip:71-84): the
 * block a scale grid of `blocks` columns implies over `ext`. */
int64_t grid_block(int64_t ext, int64_t blocks) {
    if (ext <= 0) return 1;
    if (blocks <= 1) return ext;
    const int64_t lo = (ext + blocks - 1) / blocks;
    int64_t p = 1;
    while (p < lo) p <<= 1;
    return ((ext + p - 1) / p == blocks) ? p : lo;
}

/* libref row_stride (src/r3d_gemm_mxfp4.hip:86-95): fold trailing axes until they span
 * `cols`; the next axis out is the row. */
int64_t row_stride(const RadTensor* t, int64_t cols) {
    if (!t || t->rank < 2) return cols;
    int64_t span = 1;
    for (int i = (int)t->rank - 1; i >= 0; --i) {
        if (__builtin_mul_overflow(span, t->shape[i], &span)) break;
        if (span == cols) return i > 0 ? t->stride[i - 1] : cols;
        if (span > cols) break;
    }
    return t->stride[t->rank - 2];
}

/* A row pitch the kernels can walk: not negative, and below any device allocation (the
 * reference takes the engine's strides as given; a malformed one is refused here rather
 * than turned into addresses). */
static bool pitch_ok(int64_t p) { return p >= 0 && p <= (int64_t(1) << 40); }

static bool inner_contig(const RadTensor* t) {
    return t->rank < 2 || t->stride[t->rank - 1] == 1;
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

static const int64_t kDimMax = 0x7FFFFFFLL;

int entry_preamble(const RadArgs* a, int enc, int64_t m_max, int64_t* M, int64_t* N) {
    const RadTensor* A    = rad_arg_in(a, 0);
    const RadTensor* AS   = rad_arg_in(a, 1);
    const RadTensor* B    = rad_arg_in(a, 2);
    const RadTensor* BS   = rad_arg_in(a, 3);
    const RadTensor* Y    = rad_arg_in(a, 4);
    const RadTensor* ASUM = rad_arg_in(a, 5);
    const RadTensor* BREF = rad_arg_in(a, 6);
    if (!A || !B || !BS || !Y) return RAD_E_UNSUPPORTED;
    /* a decode row takes bf16 activations without a_scale: the fused quant_act_fp8 */
    const bool fused = m_max > 0 && enc != ENC_MXFP4A16 && AS == nullptr && A->dtype == RAD_BF16;
    if (enc == ENC_MXFP4A16 ? AS != nullptr : (AS == nullptr && !fused)) return RAD_E_UNSUPPORTED;
    if (ASUM) return RAD_E_UNSUPPORTED;                 /* no zero point at any encoding */
    if (enc == ENC_FP8A8 && BREF) return RAD_E_UNSUPPORTED;   /* b_ref: e2m1 weights only */
    if (Y->dtype != RAD_BF16) return RAD_E_UNSUPPORTED;
    long long n = 0;
    if (!rad_args_geti(a, "N", &n) || n <= 0) return RAD_E_SHAPE;
    const long long yn = rad_tensor_numel(Y);
    if (yn <= 0 || yn % n) return RAD_E_SHAPE;
    if (m_max > 0 && yn / n > m_max) return RAD_E_UNSUPPORTED;   /* the band's own bound */
    if (!inner_contig(Y)) return RAD_E_STRIDE;
    *M = yn / n;
    *N = n;
    return RAD_OK;
}

int plan_mxfp4a8(const RadArgs* a, int64_t M, int64_t N, GemmPlan* P) {
    const char* dtype = rad_args_gets(a, "dtype");
    if (!dtype || strcmp(dtype, "mxfp4a8") != 0) return RAD_E_UNSUPPORTED;
    long long pb = 0;
    if (rad_args_geti(a, "pb1", &pb) && pb > 0) return RAD_E_UNSUPPORTED;   /* no parts */
    if (rad_args_geti(a, "pb2", &pb) && pb > 0) return RAD_E_UNSUPPORTED;

    const RadTensor* A  = rad_arg_in(a, 0);
    const RadTensor* AS = rad_arg_in(a, 1);
    const RadTensor* B  = rad_arg_in(a, 2);
    const RadTensor* BS = rad_arg_in(a, 3);
    const RadTensor* Y  = rad_arg_in(a, 4);
    /* AS absent with bf16 A: the decode rows' fused producer (the preamble let it through
     * only there) */
    const bool xq = A && !AS && A->dtype == RAD_BF16;
    if (!A || (!AS && !xq) || !B || !BS || !Y) return RAD_E_UNSUPPORTED;
    if ((xq ? A->dtype != RAD_BF16 : A->dtype != RAD_F8E4M3) || B->dtype != RAD_FP4E2M1 ||
        Y->dtype != RAD_BF16 || (!xq && AS->dtype != RAD_F32) ||
        (BS->dtype != RAD_E8M0 && BS->dtype != RAD_U8))
        return RAD_E_UNSUPPORTED;

    long long K = 0;
    if (!rad_args_geti(a, "K", &K)) return RAD_E_SHAPE;
    if (N <= 0 || K <= 0 || M <= 0) return RAD_E_SHAPE;
    if (M > kDimMax || N > kDimMax || K > kDimMax) return RAD_E_SHAPE;
    if (rad_tensor_numel(A) < M * K || rad_tensor_numel(B) < N * K) return RAD_E_SHAPE;
    if (xq && M > (decode_fuse(a) ? 4 : 1)) return RAD_E_UNSUPPORTED;   /* fused producer */

    /* Scale grids derived from the operands, then pinned to b 32 / a 128. */
    if (BS->rank != 2 || BS->stride[1] != 1 || BS->shape[0] < N) return RAD_E_UNSUPPORTED;
    if (!xq && (AS->rank != 2 || AS->stride[1] != 1 || AS->shape[0] < M)) return RAD_E_UNSUPPORTED;
    const int64_t bs_cols = BS->shape[1], as_cols = xq ? (K + 127) / 128 : AS->shape[1];
    if (grid_block(K, bs_cols) != 32 || grid_block(K, as_cols) != 128) return RAD_E_UNSUPPORTED;
    if (bs_cols != (K + 31) / 32 || as_cols != (K + 127) / 128) return RAD_E_UNSUPPORTED;
    if (!xq && rad_tensor_numel(AS) < M * as_cols) return RAD_E_SHAPE;

    if (!inner_contig(A) || !inner_contig(B) || !inner_contig(Y)) return RAD_E_STRIDE;
    if ((K & 1) || row_stride(B, K) != K) return RAD_E_STRIDE;   /* nibble rows packed */

    /* gfx950 gates: whole 128-wide MFMA steps.  The fast arms walk A and B in 16-byte
     * pieces and the scale plane in dwords; anything else takes the any-alignment arm
     * (the fused bf16 producer has none: the reference's rows take e4m3 A only). */
    if (K % 128) return RAD_E_UNSUPPORTED;
    const int64_t a_pitch = row_stride(A, K) * (xq ? 2 : 1);     /* bytes */
    const int64_t bs_pitch = row_stride(BS, bs_cols);
    const bool fast = aligned16(A->data) && aligned16(B->data) && !(a_pitch & 15) &&
                      !((uintptr_t)BS->data & 3) && !(bs_pitch & 3) &&
                      (xq || !((uintptr_t)AS->data & 3));
    if (!fast && xq) return RAD_E_UNSUPPORTED;

    P->enc = ENC_MXFP4A8;
    P->xq = xq;
    P->A = (const uint8_t*)A->data;
    P->AS = xq ? nullptr : (const float*)AS->data;
    P->B = (const uint8_t*)B->data;
    P->BS = BS->data;
    P->Y = (uint16_t*)Y->data;
    P->M = M; P->N = N; P->K = K;
    P->a_pitch = a_pitch;
    P->b_pitch = K / 2;
    P->y_pitch = row_stride(Y, N);
    P->as_pitch = xq ? as_cols : row_stride(AS, as_cols);
    P->bs_pitch = bs_pitch;
    P->as_cols = (int)as_cols;
    P->bs_cols = (int)bs_cols;
    P->rblk = 1;
    P->ua = fast ? 0 : UA_GEMM;
    if (!pitch_ok(P->a_pitch) || !pitch_ok(P->b_pitch) || !pitch_ok(P->y_pitch) ||
        !pitch_ok(P->as_pitch) || !pitch_ok(P->bs_pitch))
        return RAD_E_STRIDE;
    return RAD_OK;
}

int64_t mxfp4a16_scratch_bytes(int64_t M, int64_t K) {
    /* past the planes' dimension bound no plan accepts the call: -1 (never enough) */
    if (M <= 0 || K <= 0) return 0;
    if (M > kDimMax || K > kDimMax) return -1;
    return ((M * K + 255) / 256) * 256 + M * ((K + 31) / 32);
}

/* The bf16-in mxfp4 row.  Weights exactly as plan_mxfp4a8; A is bf16 [M, K] with no
 * a_scale: the launch quantises it to mxfp8 (e4m3 + E8M0 per 32 of K) in the caller's
 * scratch, so the row refuses (never overruns) a launch whose scratch is short. */
int plan_mxfp4a16(const RadArgs* a, int64_t M, int64_t N, GemmPlan* P) {
    const char* dtype = rad_args_gets(a, "dtype");
    if (!dtype || strcmp(dtype, "mxfp4a16") != 0) return RAD_E_UNSUPPORTED;
    long long pb = 0;
    if (rad_args_geti(a, "pb1", &pb) && pb > 0) return RAD_E_UNSUPPORTED;
    if (rad_args_geti(a, "pb2", &pb) && pb > 0) return RAD_E_UNSUPPORTED;

    const RadTensor* A  = rad_arg_in(a, 0);
    const RadTensor* B  = rad_arg_in(a, 2);
    const RadTensor* BS = rad_arg_in(a, 3);
    const RadTensor* Y  = rad_arg_in(a, 4);
    if (!A || !B || !BS || !Y || rad_arg_in(a, 1)) return RAD_E_UNSUPPORTED;
    if (A->dtype != RAD_BF16 || B->dtype != RAD_FP4E2M1 || Y->dtype != RAD_BF16 ||
        (BS->dtype != RAD_E8M0 && BS->dtype != RAD_U8))
        return RAD_E_UNSUPPORTED;

    long long K = 0;
    if (!rad_args_geti(a, "K", &K)) return RAD_E_SHAPE;
    if (N <= 0 || K <= 0 || M <= 0) return RAD_E_SHAPE;
    if (M > kDimMax || N > kDimMax || K > kDimMax) return RAD_E_SHAPE;
    if (rad_tensor_numel(A) < M * K || rad_tensor_numel(B) < N * K) return RAD_E_SHAPE;

    if (BS->rank != 2 || BS->stride[1] != 1 || BS->shape[0] < N) return RAD_E_UNSUPPORTED;
    const int64_t bs_cols = BS->shape[1];
    if (grid_block(K, bs_cols) != 32 || bs_cols != (K + 31) / 32) return RAD_E_UNSUPPORTED;
    long long gp = 0;   /* the group parameter must not contradict the bytes */
    if (rad_args_geti(a, "group", &gp) && gp > 0 && gp != 32) return RAD_E_SHAPE;

    if (!inner_contig(A) || !inner_contig(B) || !inner_contig(Y)) return RAD_E_STRIDE;
    if ((K & 1) || row_stride(B, K) != K) return RAD_E_STRIDE;

    if (K % 128) return RAD_E_UNSUPPORTED;
    const int64_t a_pitch = row_stride(A, K);                 /* bf16 elements */
    const int64_t bs_pitch = row_stride(BS, bs_cols);
    /* the quantiser walks A in 16-byte pieces, the GEMM B in 16-byte pieces and the scale
     * plane in dwords; anything else takes the element-wise quantiser / any-alignment GEMM */
    const bool qfast = aligned16(A->data) && !(a_pitch & 7);
    const bool gfast = aligned16(B->data) && !((uintptr_t)BS->data & 3) && !(bs_pitch & 3);
    if (!a->scratch || !aligned16(a->scratch) ||
        a->scratch_bytes < mxfp4a16_scratch_bytes(M, K))
        return RAD_E_UNSUPPORTED;

    P->enc = ENC_MXFP4A16;
    P->A = (const uint8_t*)A->data;
    P->AS = nullptr;
    P->B = (const uint8_t*)B->data;
    P->BS = BS->data;
    P->Y = (uint16_t*)Y->data;
    P->M = M; P->N = N; P->K = K;
    P->a_pitch = a_pitch;
    P->b_pitch = K / 2;
    P->y_pitch = row_stride(Y, N);
    P->as_pitch = K / 32;                                     /* of the scratch E8M0 plane */
    P->bs_pitch = bs_pitch;
    P->as_cols = (int)(K / 32);
    P->bs_cols = (int)bs_cols;
    P->rblk = 1;
    P->scratch = (uint8_t*)a->scratch;
    P->ua = (qfast ? 0 : UA_QUANT) | (gfast ? 0 : UA_GEMM);
    if (!pitch_ok(P->a_pitch) || !pitch_ok(P->b_pitch) || !pitch_ok(P->y_pitch) ||
        !pitch_ok(P->as_pitch) || !pitch_ok(P->bs_pitch))
        return RAD_E_STRIDE;
    return RAD_OK;
}

int plan_fp8a8(const RadArgs* a, int64_t M, GemmPlan* P) {
    const char* dtype = rad_args_gets(a, "dtype");
    if (!dtype || strcmp(dtype, "fp8a8") != 0) return RAD_E_UNSUPPORTED;
    long long pb = 0;
    if (rad_args_geti(a, "pb1", &pb) && pb > 0) return RAD_E_UNSUPPORTED;   /* e2m1-only parts */
    if (rad_args_geti(a, "pb2", &pb) && pb > 0) return RAD_E_UNSUPPORTED;

    const RadTensor* A  = rad_arg_in(a, 0);
    const RadTensor* AS = rad_arg_in(a, 1);
    const RadTensor* B  = rad_arg_in(a, 2);
    const RadTensor* BS = rad_arg_in(a, 3);
    const RadTensor* Y  = rad_arg_in(a, 4);
    const bool xq = A && !AS && A->dtype == RAD_BF16;       /* the decode rows' fused producer */
    if (!A || (!AS && !xq) || !B || !BS || !Y) return RAD_E_UNSUPPORTED;
    if ((xq ? A->dtype != RAD_BF16 : A->dtype != RAD_F8E4M3) || B->dtype != RAD_F8E4M3 ||
        (!xq && AS->dtype != RAD_F32) || BS->dtype != RAD_BF16 || Y->dtype != RAD_BF16)
        return RAD_E_UNSUPPORTED;

    long long N = 0, K = 0;
    if (!rad_args_geti(a, "N", &N) || !rad_args_geti(a, "K", &K)) return RAD_E_SHAPE;
    if (N <= 0 || K <= 0) return RAD_E_SHAPE;
    if (K % 128) return RAD_E_UNSUPPORTED;        /* the scale grid closes on whole blocks */
    if (M <= 0) return RAD_E_SHAPE;
    if (M > kDimMax || N > kDimMax || K > kDimMax) return RAD_E_SHAPE;
    if (rad_tensor_numel(A) < M * K || rad_tensor_numel(B) < N * K) return RAD_E_SHAPE;
    if (xq && M > (decode_fuse(a) ? 4 : 1)) return RAD_E_UNSUPPORTED;   /* fused producer */

    if (BS->rank != 2 || BS->stride[1] != 1) return RAD_E_UNSUPPORTED;
    if (!xq && (AS->rank != 2 || AS->stride[1] != 1 || AS->shape[0] < M)) return RAD_E_UNSUPPORTED;
    const int64_t bs_cols = BS->shape[1], as_cols = xq ? (K + 127) / 128 : AS->shape[1];
    if (grid_block(K, bs_cols) != 128 || grid_block(K, as_cols) != 128) return RAD_E_UNSUPPORTED;
    if (bs_cols != (K + 127) / 128 || as_cols != (K + 127) / 128) return RAD_E_SHAPE;
    if (!xq && rad_tensor_numel(AS) < M * as_cols) return RAD_E_SHAPE;
    int rblk;
    if (BS->shape[0] >= N) {
        if (BS->shape[0] != N) return RAD_E_SHAPE;
        rblk = 1;                                  /* per-row grid */
    } else {
        if (grid_block(N, BS->shape[0]) != 128 || BS->shape[0] != (N + 127) / 128)
            return RAD_E_UNSUPPORTED;
        rblk = 128;                                /* 128 x 128 checkpoint block grid */
    }
    if (rad_tensor_numel(BS) < (rblk > 1 ? (N + 127) / 128 : N) * bs_cols) return RAD_E_SHAPE;

    long long gp = 0;   /* the group parameter must not contradict the bytes */
    if (rad_args_geti(a, "group", &gp) && gp > 0 && gp != 128) return RAD_E_SHAPE;

    if (!inner_contig(A) || !inner_contig(B) || !inner_contig(Y)) return RAD_E_STRIDE;

    /* the fast arms walk A and B in 16-byte pieces; anything else takes the any-alignment
     * arm (the fused bf16 producer has none: the reference's rows take e4m3 A only) */
    const int64_t a_pitch = row_stride(A, K) * (xq ? 2 : 1), b_pitch = row_stride(B, K);
    const bool fast = aligned16(A->data) && aligned16(B->data) && !(a_pitch & 15) &&
                      !(b_pitch & 15) && !((uintptr_t)BS->data & 1) &&
                      (xq || !((uintptr_t)AS->data & 3));
    if (!fast && xq) return RAD_E_UNSUPPORTED;

    P->enc = ENC_FP8A8;
    P->xq = xq;
    P->A = (const uint8_t*)A->data;
    P->AS = xq ? nullptr : (const float*)AS->data;
    P->B = (const uint8_t*)B->data;
    P->BS = BS->data;
    P->Y = (uint16_t*)Y->data;
    P->M = M; P->N = N; P->K = K;
    P->a_pitch = a_pitch;
    P->b_pitch = b_pitch;
    P->y_pitch = row_stride(Y, N);
    P->as_pitch = xq ? as_cols : row_stride(AS, as_cols);
    P->bs_pitch = row_stride(BS, bs_cols);
    P->as_cols = (int)as_cols;
    P->bs_cols = (int)bs_cols;
    P->rblk = rblk;
    P->ua = fast ? 0 : UA_GEMM;
    if (!pitch_ok(P->a_pitch) || !pitch_ok(P->b_pitch) || !pitch_ok(P->y_pitch) ||
        !pitch_ok(P->as_pitch) || !pitch_ok(P->bs_pitch))
        return RAD_E_STRIDE;
    return RAD_OK;
}

/* Decode geometry: a 16-row weight tile is one wave per K chunk; the chunks of a tile share
 * a workgroup (LDS fold in chunk order).  Waves per workgroup come from the LDS budget of
 * one wave's run buffers (160 KB per CU). */
void decode_geom(int64_t M, int64_t N, int64_t K, int64_t force_chunks, DecodeGeom* g,
                 int wave_lds) {
    g->mt = M <= 1 ? 1 : M <= 4 ? 4 : 16;          /* rounds UP: every row is written */
    g->steps = (int)(K / 128);
    g->tiles = (N + 15) / 16;
    /* waves one workgroup can hold in 160 KB of LDS, as a power of two <= 8 */
    int maxw = 8;
    if (wave_lds > 0) {
        const int fit = (160 * 1024) / wave_lds;
        maxw = fit >= 8 ? 8 : fit >= 4 ? 4 : fit >= 2 ? 2 : 1;
    }
    int c = 1;
    if (force_chunks > 0) {
        c = force_chunks >= 8 ? 8 : force_chunks >= 4 ? 4 : force_chunks >= 2 ? 2 : 1;
    } else {
        /* measured on MI355X at the 27B-class shapes: two chunks per tile wins wherever a
         * chunk keeps >= 8 steps (more resident waves, each still many runs long); more
         * only when the tile count is small */
        if (g->steps >= 16) c = 2;
        while (c < 8 && g->tiles * c < 512 && g->steps / (2 * c) >= 8) c *= 2;
    }
    if (c > maxw) c = maxw;
    while (c > 1 && c > g->steps) c >>= 1;
    g->chunks = c;
    const int w0 = maxw < 4 ? maxw : 4;
    g->waves = c > w0 ? c : w0;
    g->tiles_per_block = g->waves / c;
    g->blocks = (g->tiles + g->tiles_per_block - 1) / g->tiles_per_block;
}

bool quad_fits(const GemmPlan& P) {
    const int64_t lim = (int64_t)1 << 31;
    return 8 * P.b_pitch < lim && P.a_pitch < lim && P.as_pitch < lim && P.bs_pitch < lim;
}

/* Quad geometry: split K until about env_quad_waves() waves are in flight (default 2048
 * at one activation row, 1280 at 2..4), keeping >= 16 groups per chunk.  A split doubles
 * the workgroups, and every workgroup stages the whole-K activation rows: at four rows
 * those are as many bytes as a quarter of its weights (o, K = 4096 N = 5376, M = 4: 5.28 us
 * unsplit against 6.11 split in two), while one row is cheap enough that more waves pay
 * (C2 down, K = 21504 N = 5376, M = 1: 12.73 split against 13.06). */
bool quad_geom(int enc, int64_t M, int64_t N, int64_t K, int64_t force_chunks, QuadGeom* g,
               int xq) {
    if (M < 1 || M > 4 || N < 1 || K < 128 || K % 128 != 0) return false;
    if (force_chunks > 0 && force_chunks != 1 && force_chunks != 2 && force_chunks != 4)
        return false;
    g->mt = M <= 1 ? 1 : 4;
    g->qpw = env_quad_qpw();
    g->groups = (int)(K / 128);
    g->quads = (N + 3) / 4;
    g->nblk = (N + 4 * g->qpw - 1) / (4 * g->qpw);
    const int64_t target = env_quad_waves() > 0 ? env_quad_waves() : g->mt == 1 ? 2048 : 1280;
    int c = 1;
    if (force_chunks > 0) {
        c = (int)force_chunks;
    } else {
        while (c < 4 && g->nblk * c < target && g->groups >= 16 * c) c *= 2;
    }
    while (c > 1 && c > g->groups) c >>= 1;
    g->chunks = c;
    /* eight waves share one activation staging: measured on MI355X, a gain at MT = 4 (the
     * staging is four rows; 2-4 % on config 2/4 shapes) and for fp8a8 at MT = 1 without a
     * K split (1.5 % at config 1), a loss for mxfp4a8 at MT = 1 (the long-K split shape
     * most: 13.2 -> 15.5 us) except with the fused producer, whose bf16 re-read it halves
     * (15.0 -> 14.4 us at config 2's gate_up); two quads a wave keep four waves */
    /* R3D_GFX950_QWV = 7 only where the kernel has a seven-wave form: no K split, no fused
     * producer (elsewhere the policy decides, as without the lever) */
    int wv_env = env_quad_wv();
    if (wv_env == 7 && (c != 1 || xq || g->qpw != 1)) wv_env = 0;
    g->gmax = (g->groups + c - 1) / c;
    /* LDS of a workgroup of wv waves (quad_lds, the layout the kernel computes too) */
    auto lds_of = [&](int wv) { return quad_lds(enc, g->mt, g->qpw, wv, K, c).lds; };
    g->wv = g->qpw == 2 ? 4 : wv_env ? wv_env
          : (g->mt == 4 || (enc == ENC_FP8A8 && c == 1) || xq) ? 8 : 4;
    if (g->qpw == 1 && c == 1 && !xq && !wv_env) {
        /* seven waves when that evens the workgroups over the CUs: the most waves any CU
         * holds, ceil(blocks / 256) x waves, is what the stream waits for (config 1: 768
         * workgroups of 7 = 21 a CU against 672 of 8 = 24; config 2's gate_up at M = 1:
         * against 1344 of 4, also 24) */
        const int w0 = g->wv;
        const int64_t b0 = (g->nblk + w0 - 1) / w0, b7 = (g->nblk + 6) / 7;
        if (((b7 + 255) / 256) * 7 < ((b0 + 255) / 256) * w0 && lds_of(7) <= kQuadMaxLds)
            g->wv = 7;
    }
    /* the policy's seven or eight waves only where their LDS fits; four otherwise (a lever
     * that does not fit refuses, so the next kernel runs) */
    if (!wv_env && g->wv != 4 && lds_of(g->wv) > kQuadMaxLds) g->wv = 4;
    g->bpb = g->wv / c;
    g->blocks = (g->nblk + g->bpb - 1) / g->bpb;
    {
        /* the deepest supported ring that no wave's step count falls below */
        static const int kDepths[] = {8, 4, 2, 1};
        const int ns_min = (g->groups / c + 3) / 4;
        /* four steps, or eight at mxfp4a8 where every wave walks 16+ steps (one 1 KB load
         * a step, so eight fit its registers at full occupancy): C2 down at M = 1, 21 steps
         * a chunk, 12.86 -> 12.59 us; at 11 steps (gate_up, config 1) two to eight tie */
        const int want = env_quad_depth(enc) > 0 ? env_quad_depth(enc)
                       : enc == ENC_MXFP4A8 && ns_min >= 16 ? 8 : 4;
        g->depth = 1;
        for (int d : kDepths)
            if (d <= want && d <= ns_min) { g->depth = d; break; }
    }
    const QuadLds ql = quad_lds(enc, g->mt, g->qpw, g->wv, K, c);
    if (ql.lds > kQuadMaxLds || g->blocks > 0x7FFFFFFF) return false;
    g->xs_off = (int)ql.xs_off;
    g->sc_off = (int)ql.sc_off;
    g->sc_bytes = (int)ql.sc_bytes;
    g->lds = (int)ql.lds;
    return true;
}

bool lines_fits(const GemmPlan& P) {
    const int64_t lim = (int64_t)1 << 31;
    return 64 * P.b_pitch < lim && (P.M - 1) * P.a_pitch + P.K < lim;   /* up to 4 tiles */
}

/* Line geometry: tw tiles per wave (policy or R3D_GFX950_LTW), then split K until about
 * env_lines_waves() waves are in flight (keeping >= 4 lines per chunk), or until a wave's
 * scale tables fit the LDS budget. */
bool lines_geom(int enc, int64_t M, int64_t N, int64_t K, int64_t force_chunks, LinesGeom* g) {
    /* M <= 4 shapes the quad GEMV cannot stage run faster on the 16-row GEMV's 4-row
     * instantiation (measured on MI355X at K = 21504) */
    if (M < 5 || M > 16 || N < 1 || K < 128 || K % 128 != 0) return false;
    if (enc != ENC_MXFP4A8 && enc != ENC_FP8A8) return false;
    if (force_chunks > 0 && force_chunks != 1 && force_chunks != 2 && force_chunks != 4)
        return false;
    const int G = enc == ENC_MXFP4A8 ? 2 : 1;
    g->mt = M <= 8 ? 8 : 16;
    g->groups = (int)(K / 128);
    g->units = (g->groups + G - 1) / G;
    g->tiles = (N + 15) / 16;
    /* two tiles per wave halve the activation loads per weight byte; measured best on
     * MI355X at the 27B-class shapes (M = 8..16) */
    const int etw = env_lines_tw();
    g->tw = etw == 1 || etw == 2 || etw == 4 ? etw : 2;
    g->nblk = (g->tiles + g->tw - 1) / g->tw;
    auto wlds_of = [&](int c) { return lines_wlds(enc, g->tw, K, c); };
    int c = 1;
    if (force_chunks > 0) {
        c = (int)force_chunks;
    } else {
        const int64_t target = env_lines_waves();
        while (c < 4 && g->units >= 8 * c &&
               (g->nblk * c < target || 4 * wlds_of(c) > kLinesMaxLds))
            c *= 2;
    }
    while (c > 1 && c > g->units) c >>= 1;
    g->chunks = c;
    g->tpb = 4 / c;
    g->blocks = (g->nblk + g->tpb - 1) / g->tpb;
    g->gmax = G * ((g->units + c - 1) / c);
    g->wlds = wlds_of(c);
    const int fold = 4 * 1024 * g->tw;
    g->lds = 4 * g->wlds > fold ? 4 * g->wlds : fold;
    {
        static const int kDepths[] = {4, 2, 1};
        const int ns_min = g->units / c;
        const int ed = env_lines_depth();
        int want = ed > 0 ? ed : (g->tw >= 2 ? 2 : 4);   /* measured best */
        if (g->tw >= 4 && want > 2) want = 2;             /* register budget */
        g->depth = 1;
        for (int d : kDepths)
            if (d <= want && d <= ns_min) { g->depth = d; break; }
    }
    return g->lds <= kLinesMaxLds && g->blocks <= 0x7FFFFFFF;
}

/* Prefill tile choice: 64 wmw tokens (4 fragments per wave; 2 with e4m3 weights, whose
 * 8-register operands, row scales and flush results fill the register file at 4 x 2) by
 * 32 wnf weight rows.  Workgroups run one per CU, so the launch
 * takes ceil(tiles / ncu) rounds; a round costs about wnf + 1/2 fragment-steps (the
 * fixed activation reads of a step).  The cheapest total wins, ties to the larger tile. */
/* R3D_GFX950_F8_TILE: "128" keeps the e4m3 prefill on the 128 x 128 tile at every M,
 * "256" takes the 128 x 256 tile at every M past 128 (default: by round cost) */
static int f8_tile_lever() {
    static const int v = [] {
        const char* e = getenv("R3D_GFX950_F8_TILE");
        return e && strcmp(e, "128") == 0 ? 128 : e && strcmp(e, "256") == 0 ? 256 : 0;
    }();
    return v;
}

void prefill_geom(int64_t M, int64_t N, int64_t K, int mode, int ncu, PrefillGeom* g) {
    /* e4m3 weights: two 8-register operand sets, the row scales and two f32 result sets per
     * fragment hold the tile at 4 fragment pairs (at 6, 185 registers spill) */
    static const int kWnf[] = {8, 7, 6, 4};
    static const int kWnfF8[] = {4};
    /* up to 128 tokens the f32-a_scale mode runs 2 token fragments per wave (the 4-fragment
     * tile would leave most of its MFMAs on padding rows): 33 against 45 us at M = 8..64 */
    const bool narrow = mode == PF_F8 || (mode == PF_A8 && M <= 128);
    const int wmw = narrow ? 2 : 4;
    if (ncu <= 0) ncu = 256;
    int best = 0;
    double best_cost = 0.0;
    auto consider = [&](int w) {
        const int64_t tiles = ((N + 32 * w - 1) / (32 * w)) * ((M + 64 * wmw - 1) / (64 * wmw));
        const double cost = (double)((tiles + ncu - 1) / ncu) * (w + 0.5);
        if (best == 0 || cost < best_cost) { best = w; best_cost = cost; }
    };
    if (narrow)
        for (int w : kWnfF8) consider(w);
    else
        for (int w : kWnf) consider(w);
    g->wnf = best;
    g->wmf = wmw;
    g->nst = 3;
    g->wv = 8;
    /* e4m3 weights past 128 tokens: four waves (one a SIMD, 512 registers each) hold a
     * 128 x 256 tile -- a quarter fewer bytes per MFMA than the 128 x 128 tile.  A round of
     * those tiles takes 1.71x a round of 128 x 128 tiles (config 3's shape: 387 us over 6
     * rounds against 416 over 11), so it runs where its rounds cost less. */
    if (mode == PF_F8 && M > 128 && f8_tile_lever() != 128) {
        const int64_t rn = (N + 127) / 128;
        const int64_t r8 = (rn * ((M + 127) / 128) + ncu - 1) / ncu;
        int64_t c4 = 171 * ((rn * ((M + 255) / 256) + ncu - 1) / ncu);
        if (const int64_t n1 = prefill_f8_split_n(M, N, ncu)) {   /* whole rounds + remainder */
            const int64_t r1 = ((n1 / 128) * ((M + 255) / 256) + ncu - 1) / ncu;
            const int64_t r2 = (((N - n1 + 127) / 128) * ((M + 127) / 128) + ncu - 1) / ncu;
            c4 = 171 * r1 + 100 * r2;
        }
        if (f8_tile_lever() == 256 || c4 < 100 * r8) {
            g->wnf = 4;
            g->wmf = 8;
            g->wv = 4;
        }
    }
    g->bn = 32 * g->wnf;
    g->bm = 8 * g->wv * g->wmf;
    g->grid_m = (M + g->bm - 1) / g->bm;
    g->grid_n = (N + g->bn - 1) / g->bn;
    g->tiles = g->grid_m * g->grid_n;
    g->steps = (int)(K / 128);
    g->lds = g->nst * prefill_stage_bytes(g->wnf, g->wmf, mode == PF_F8 ? 2 : 1, g->wv);
}

int64_t prefill_f8_split_n(int64_t M, int64_t N, int ncu) {
    if (ncu <= 0) ncu = 256;
    if (M <= 128 || N <= 128) return 0;
    const int64_t rn = (N + 127) / 128, mt = (M + 255) / 256;
    const int64_t tiles = rn * mt;
    const int64_t whole = tiles / ncu;                  /* whole rounds of the wide tile */
    if (whole < 1 || tiles % ncu == 0) return 0;
    const int64_t n1t = whole * ncu / mt;               /* weight tiles inside them */
    if (n1t < 1 || n1t >= rn) return 0;
    const int64_t t2 = ((N - 128 * n1t + 127) / 128) * ((M + 127) / 128);
    const int64_t r1 = (n1t * mt + ncu - 1) / ncu, r2 = (t2 + ncu - 1) / ncu;
    const int64_t rall = (tiles + ncu - 1) / ncu;
    return 171 * r1 + 100 * r2 < 171 * rall ? 128 * n1t : 0;
}

int skinny_passes(int enc, int64_t M, int64_t N, int ncu) {
    if ((enc != ENC_MXFP4A8 && enc != ENC_FP8A8) || M < 17 || M > 64) return 0;
    static const int lever = [] {
        const char* e = getenv("R3D_GFX950_SKINNY");
        return e ? (atoi(e) ? 1 : 0) : -1;
    }();
    if (lever >= 0) return lever ? (int)((M + 15) / 16) : 0;
    if (ncu <= 0) ncu = 256;
    const int64_t tiles = (N + 127) / 128;            /* the narrow (128 x 128) prefill tile */
    const int64_t act = tiles < ncu ? tiles : ncu;
    const int passes = (int)((M + 15) / 16);
    return passes * act < 300 ? passes : 0;
}

int tile_splitk(int enc, int64_t M, int64_t N, int64_t K, int ncu, int* cst, PrefillGeom* g) {
    if ((enc != ENC_MXFP4A8 && enc != ENC_FP8A8) || M < 1 || M > 128 || N < 1 || K < 128)
        return 0;
    static const long long lever = [] {
        const char* e = getenv("R3D_GFX950_SPLITK_UNITS");
        return e ? atoll(e) : -1LL;
    }();
    if (ncu <= 0) ncu = 256;
    const int64_t target = lever >= 0 ? lever : ncu;
    /* the split's tile: 64 tokens up to M = 64 (256 e2m1 / 128 e4m3 weight rows), else
     * 128 x 128 */
    const int wmf = M <= 64 ? 1 : 2;
    const int wnf = enc == ENC_MXFP4A8 && wmf == 1 ? 8 : 4;
    const int64_t bn = 32 * wnf;
    const int64_t tiles = (N + bn - 1) / bn;
    const int64_t steps = K / 128;
    int64_t kc = target / tiles;
    if (kc > steps / kSplitMinSteps) kc = steps / kSplitMinSteps;
    if (kc < 2 || tiles * kc > 0x7FFFFFFF) return 0;
    const int64_t c = (steps + kc - 1) / kc;
    kc = (steps + c - 1) / c;                           /* no empty chunk */
    if (kc < 2) return 0;
    if (cst) *cst = (int)c;
    if (g) {
        g->wnf = wnf;
        g->wmf = wmf;
        g->nst = 3;
        g->wv = 8;
        g->bn = (int)bn;
        g->bm = 64 * wmf;
        g->grid_m = 1;
        g->grid_n = tiles;
        g->tiles = tiles;
        g->steps = (int)steps;
        g->lds = g->nst * prefill_stage_bytes(wnf, wmf, enc == ENC_FP8A8 ? 2 : 1);
    }
    return (int)kc;
}

/* The skinny-band GEMV's geometry for a K split of at most kc0 chunks: the chunk (cg
 * groups, a whole number of 128-byte lines) as long as the LDS budget allows. */
static bool wide_geom(int enc, int64_t M, int64_t N, int64_t K, int64_t kc0, WideGeom* w) {
    const int G = enc == ENC_MXFP4A8 ? 2 : 1;
    const int64_t steps = K / 128;
    w->tw = 2;
    w->ntg = (int)((M + 15) / 16);
    w->ntiles = (N + 255) / 256;
    int64_t cg = (steps + kc0 - 1) / kc0;
    cg = (cg + G - 1) / G * G;
    auto lds_of = [&](int64_t c, int64_t* sc) {
        const int64_t scl = (16 * w->tw * c * 4 + 255) / 256 * 256;
        if (sc) *sc = scl;
        return c * w->ntg * 2048 + c * 256 + 8 * scl;
    };
    while (cg > G && lds_of(cg, nullptr) > kWideMaxLds) cg -= G;
    int64_t scl = 0;
    const int64_t lds = lds_of(cg, &scl);
    if (lds > kWideMaxLds) return false;
    w->cg = (int)cg;
    w->sclds = (int)scl;
    w->lds = (int)lds;
    w->d = 1;
    return true;
}

int splitk_plan(int enc, int64_t M, int64_t N, int64_t K, int ncu, int* kc, int* cst,
                PrefillGeom* g, WideGeom* w) {
    if ((enc != ENC_MXFP4A8 && enc != ENC_FP8A8) || M < 1 || M > 128 || N < 1 || K < 128)
        return 0;
    static const bool tile_only = [] {
        const char* e = getenv("R3D_GFX950_SPLITK_KERNEL");
        return e && strcmp(e, "tile") == 0;
    }();
    if (M > 64 || tile_only) {
        int c = 0;
        const int k = tile_splitk(enc, M, N, K, ncu, &c, g);
        if (!k) return 0;
        if (kc) *kc = k;
        if (cst) *cst = c;
        return 2;
    }
    static const long long lever = [] {
        const char* e = getenv("R3D_GFX950_SPLITK_UNITS");
        return e ? atoll(e) : -1LL;
    }();
    if (ncu <= 0) ncu = 256;
    const int64_t target = lever >= 0 ? lever : ncu;
    /* units aim at the target over the GEMV's 256-row tiles, at least kSplitMinSteps groups a
     * chunk; the LDS budget may shorten the chunk (more chunks) */
    const int64_t steps = K / 128;
    const int64_t ntiles = (N + 255) / 256;
    int64_t kc0 = target / ntiles;
    if (kc0 > steps / kSplitMinSteps) kc0 = steps / kSplitMinSteps;
    if (kc0 < 2) return 0;
    WideGeom tmp{};
    WideGeom* wg = w ? w : &tmp;
    if (!wide_geom(enc, M, N, K, kc0, wg)) return 0;
    const int64_t kcw = (steps + wg->cg - 1) / wg->cg;
    if (kcw < 2 || wg->ntiles * kcw > 0x7FFFFFFF) return 0;
    if (kc) *kc = (int)kcw;
    if (cst) *cst = wg->cg;
    return 1;
}

int64_t tile_splitk_bytes(int enc, int64_t M, int64_t N, int64_t K, int ncu) {
    int kc = 0;
    return splitk_plan(enc, M, N, K, ncu, &kc, nullptr, nullptr, nullptr) ? (int64_t)kc * M * N * 4 : 0;
}

int64_t tile_scratch_bytes(const RadArgs* a, int enc, int ncu) {
    long long N = 0, K = 0, M = 0;
    if (!rad_args_geti(a, "N", &N) || !rad_args_geti(a, "K", &K)) return 0;
    if (N <= 0 || K <= 0 || N > (1LL << 34) || K > (1LL << 27)) return 0;
    /* the launch's own M (numel(y) / N) when y is there, else the M parameter, else the
     * largest M the split takes */
    const RadTensor* Y = rad_arg_in(a, 4);
    const long long yn = Y ? rad_tensor_numel(Y) : 0;
    if (yn > 0 && yn % N == 0)
        M = yn / N;
    else if (!rad_args_geti(a, "M", &M) || M <= 0)
        M = 128;
    return tile_splitk_bytes(enc, M, N, K, ncu);
}

int decode_split_plan(int enc, int64_t M, int64_t N, int64_t K, int ncu, bool quad, int64_t pin,
                      int* kc, WideGeom* w) {
    if (quad || pin > 0 || M < 1 || M > 16 || N < 1 || K < 1 || N * K < kDecodeSplitMinWeights)
        return 0;
    int cst = 0;
    return splitk_plan(enc, M, N, K, ncu, kc, &cst, nullptr, w) == 1 ? 1 : 0;
}

int64_t decode_scratch_bytes(const RadArgs* a, int enc, int ncu) {
    long long N = 0, K = 0, M = 0;
    if (!rad_args_geti(a, "N", &N) || !rad_args_geti(a, "K", &K)) return 0;
    if (N <= 0 || K <= 0 || N > (1LL << 34) || K > (1LL << 27)) return 0;
    const RadTensor* Y = rad_arg_in(a, 4);
    const long long yn = Y ? rad_tensor_numel(Y) : 0;
    if (yn > 0 && yn % N == 0)
        M = yn / N;
    else if (!rad_args_geti(a, "M", &M) || M <= 0)
        M = 16;
    if (M > 16) return 0;
    const int64_t pin = decode_splitk(a);
    QuadGeom qg{};
    const bool quad = quad_geom(enc, M, N, K, pin, &qg, false);
    int kc = 0;
    return decode_split_plan(enc, M, N, K, ncu, quad, pin, &kc, nullptr) ? (int64_t)kc * M * N * 4
                                                                          : 0;
}

int band_row_pitch(const RadTensor* t, int64_t cols, int64_t* pitch) {
    if (!t || !t->data) return -1;
    if (t->rank == 1) {
        if (rad_tensor_numel(t) != cols || t->stride[0] != 1) return -2;
        *pitch = 0;
        return 0;
    }
    if (t->rank == 2) {
        if (t->stride[1] != 1) return -3;
        *pitch = t->shape[1] == cols ? t->stride[0] : cols;
        return pitch_ok(*pitch) ? 0 : -4;         /* a walkable pitch (not in the reference) */
    }
    if (t->rank >= 3) {
        if (t->stride[t->rank - 1] != 1) return -3;
        if (t->shape[t->rank - 1] != cols) { *pitch = cols; return 0; }
        for (int i = 0; i < (int)t->rank - 1; ++i) {
            int64_t span = 0;
            if (__builtin_mul_overflow(t->shape[i + 1], t->stride[i + 1], &span) ||
                t->stride[i] != span)
                return -4;
        }
        *pitch = cols;
        return 0;
    }
    return -1;                                   /* rank 0 */
}

int plan_quant_act_fp8(const RadArgs* a, QuantPlan* P) {
    const RadTensor* x = rad_arg_in(a, 0);
    const RadTensor* q = rad_arg_in(a, 1);
    const RadTensor* sc = rad_arg_in(a, 2);
    if (!x || !q || !sc) return RAD_E_INVAL;
    if (x->dtype != RAD_F32 && x->dtype != RAD_BF16) return RAD_E_DTYPE;
    if (q->dtype != RAD_F8E4M3 || sc->dtype != RAD_F32) return RAD_E_DTYPE;
    long long v = 0;
    const int64_t n = rad_args_geti(a, "n", &v) ? (int64_t)v : (x->rank >= 2 ? x->shape[1] : 0);
    if (n <= 0 || n > kDimMax) return RAD_E_SHAPE;
    const int64_t rows = rad_tensor_numel(x) / n;
    if (rows <= 0 || rows > 0xffff) return RAD_E_SHAPE;
    int64_t g = rad_args_geti(a, "group", &v) ? (int64_t)v : n;
    if (g <= 0 || g > n) g = n;
    const int64_t ngrp = (n + g - 1) / g;
    if (ngrp > 0x7fffffffLL) return RAD_E_SHAPE;
    if (rad_tensor_numel(q) < rows * n || rad_tensor_numel(sc) < rows * ngrp) return RAD_E_SHAPE;
    int64_t xp = 0, qp = 0, sp = 0;
    if (band_row_pitch(x, n, &xp) || band_row_pitch(q, n, &qp) || band_row_pitch(sc, ngrp, &sp))
        return RAD_E_STRIDE;
    P->x = (const uint8_t*)x->data;
    P->q = (uint8_t*)q->data;
    P->scale = (float*)sc->data;
    P->x_bf16 = x->dtype == RAD_BF16;
    P->rows = rows;
    P->n = n;
    P->g = g;
    P->ngrp = ngrp;
    P->x_pitch = xp;
    P->q_pitch = qp;
    P->s_pitch = sp;
    return RAD_OK;
}

int plan_gated_quant_fp8(const RadArgs* a, GatedPlan* P) {
    const RadTensor* gu = rad_arg_in(a, 0);
    const RadTensor* q = rad_arg_in(a, 1);
    const RadTensor* sc = rad_arg_in(a, 2);
    const RadTensor* ob = rad_arg_in(a, 3);
    if (!gu || !q || !sc) return RAD_E_INVAL;
    if (gu->dtype != RAD_F32 && gu->dtype != RAD_BF16) return RAD_E_DTYPE;
    if (q->dtype != RAD_F8E4M3 || sc->dtype != RAD_F32) return RAD_E_DTYPE;
    if (ob && ob->dtype != RAD_F32 && ob->dtype != RAD_BF16) return RAD_E_DTYPE;
    long long v = 0;
    const int64_t n = rad_args_geti(a, "n", &v) ? (int64_t)v
                                                : (gu->rank >= 2 ? gu->shape[1] / 2 : 0);
    if (n <= 0 || n > kDimMax) return RAD_E_SHAPE;
    const char* act = rad_args_gets(a, "act");
    int64_t g = rad_args_geti(a, "group", &v) ? (int64_t)v : n;
    if (g <= 0 || g > n) g = n;
    const int64_t ngrp = (n + g - 1) / g;
    const int64_t rows = rad_tensor_numel(gu) / (2 * n);
    if (rows <= 0 || rows > 0xffff) return RAD_E_SHAPE;
    if (rad_tensor_numel(q) < rows * n || rad_tensor_numel(sc) < rows * ngrp) return RAD_E_SHAPE;
    if (ob && rad_tensor_numel(ob) < rows * n) return RAD_E_SHAPE;
    int64_t gp = 0, qp = 0, sp = 0, op = 0;
    if (band_row_pitch(gu, 2 * n, &gp) || band_row_pitch(q, n, &qp) ||
        band_row_pitch(sc, ngrp, &sp) || (ob && band_row_pitch(ob, n, &op)))
        return RAD_E_STRIDE;
    P->gu = (const uint8_t*)gu->data;
    P->q = (uint8_t*)q->data;
    P->scale = (float*)sc->data;
    P->ob = ob ? (uint8_t*)ob->data : nullptr;
    P->gu_bf16 = gu->dtype == RAD_BF16;
    P->ob_bf16 = ob && ob->dtype == RAD_BF16;
    P->silu = !act || strcmp(act, "sigmoid") != 0;
    P->rows = rows;
    P->n = n;
    P->g = g;
    P->ngrp = ngrp;
    P->gu_pitch = gp;
    P->q_pitch = qp;
    P->s_pitch = sp;
    P->ob_pitch = op;
    return RAD_OK;
}

int plan_rmsnorm_quant_fp8(const RadArgs* a, RmsPlan* P) {
    if (!a || a->n_t < 5) return RAD_E_INVAL;
    const RadTensor* x = rad_arg_in(a, 0);
    const RadTensor* res = rad_arg_in(a, 1);
    const RadTensor* w = rad_arg_in(a, 2);
    const RadTensor* q = rad_arg_in(a, 3);
    const RadTensor* sc = rad_arg_in(a, 4);
    const RadTensor* ob = rad_arg_in(a, 5);
    if (!x || !w || !q || !sc) return RAD_E_INVAL;
    if (x->dtype != RAD_BF16) return RAD_E_DTYPE;
    if (res && res->dtype != RAD_BF16) return RAD_E_DTYPE;
    if (w->dtype != RAD_F32 && w->dtype != RAD_BF16) return RAD_E_DTYPE;
    if (q->dtype != RAD_F8E4M3 || sc->dtype != RAD_F32) return RAD_E_DTYPE;
    if (ob && ob->dtype != RAD_F32 && ob->dtype != RAD_BF16) return RAD_E_DTYPE;
    long long v = 0;
    const int64_t n = rad_args_geti(a, "n", &v) ? (int64_t)v
                                                : (w->rank ? w->shape[w->rank - 1] : 0);
    if (n <= 0 || n > 30720) return RAD_E_SHAPE;
    int64_t g = rad_args_geti(a, "group", &v) ? (int64_t)v : 0;
    if (g <= 0 || g > n) g = n;
    const int64_t ngrp = (n + g - 1) / g;
    const int64_t rows = rad_tensor_numel(x) / n;
    if (rows <= 0 || rows > 0xffff) return RAD_E_SHAPE;
    if (rad_tensor_numel(q) < rows * n || rad_tensor_numel(sc) < rows * ngrp ||
        rad_tensor_numel(w) < n)
        return RAD_E_SHAPE;
    if (res && rad_tensor_numel(res) < rows * n) return RAD_E_SHAPE;
    if (ob && rad_tensor_numel(ob) < rows * n) return RAD_E_SHAPE;
    int64_t xp = 0, rp = 0, qp = 0, sp = 0, op = 0;
    if (band_row_pitch(x, n, &xp)) return RAD_E_STRIDE;
    if (res && band_row_pitch(res, n, &rp)) return RAD_E_STRIDE;
    if (w->rank != 1 || w->stride[0] != 1) return RAD_E_STRIDE;
    if (band_row_pitch(q, n, &qp) || band_row_pitch(sc, ngrp, &sp)) return RAD_E_STRIDE;
    if (ob && band_row_pitch(ob, n, &op)) return RAD_E_STRIDE;
    P->x = (const uint8_t*)x->data;
    P->res = res ? (uint8_t*)res->data : nullptr;
    P->w = (const uint8_t*)w->data;
    P->q = (uint8_t*)q->data;
    P->scale = (float*)sc->data;
    P->ob = ob ? (uint8_t*)ob->data : nullptr;
    P->w_bf16 = w->dtype == RAD_BF16;
    P->ob_bf16 = ob && ob->dtype == RAD_BF16;
    P->rows = rows;
    P->n = n;
    P->g = g;
    P->ngrp = ngrp;
    P->x_pitch = xp;
    P->r_pitch = rp;
    P->q_pitch = qp;
    P->s_pitch = sp;
    P->ob_pitch = op;
    P->eps = (float)rad_args_getf_or(a, "eps", 1e-6);
    P->wadd = (float)rad_args_getf_or(a, "wadd", 0.0);
    return RAD_OK;
}

int64_t gemm_gated_scratch_bytes(const RadArgs* a) {
    long long N = 0;
    if (!rad_args_geti(a, "N", &N) || N <= 0 || N > (1LL << 34)) return 0;
    return 64 * (int64_t)N * 2;
}

int plan_gemm_gated(const RadArgs* a, GemmPlan* G, GatedPlan* E) {
    if (env_no_fp8a8()) return RAD_E_UNSUPPORTED;
    const RadTensor* A = rad_arg_in(a, 0);
    const RadTensor* AS = rad_arg_in(a, 1);
    const RadTensor* B = rad_arg_in(a, 2);
    const RadTensor* BS = rad_arg_in(a, 3);
    const RadTensor* Q = rad_arg_in(a, 4);
    const RadTensor* SC = rad_arg_in(a, 5);
    const RadTensor* OB = rad_arg_in(a, 6);
    if (!A || !AS || !B || !BS || !Q || !SC) return RAD_E_UNSUPPORTED;
    if (rad_arg_in(a, 7)) return RAD_E_UNSUPPORTED;              /* a_sum */
    if (Q->dtype != RAD_F8E4M3 || SC->dtype != RAD_F32) return RAD_E_UNSUPPORTED;
    if (OB && OB->dtype != RAD_BF16 && OB->dtype != RAD_F32) return RAD_E_UNSUPPORTED;
    /* act is required here: a row may compile one gate only */
    const char* act = rad_args_gets(a, "act");
    if (!act || (strcmp(act, "silu") != 0 && strcmp(act, "sigmoid") != 0))
        return RAD_E_UNSUPPORTED;
    long long N = 0;
    if (!rad_args_geti(a, "N", &N) || N <= 0 || (N & 1)) return RAD_E_SHAPE;
    const int64_t n = N / 2;
    long long gv = 0;
    int64_t g = rad_args_geti(a, "group", &gv) && gv > 0 ? (int64_t)gv : n;
    if (g > n) g = n;
    const int64_t ngrp = (n + g - 1) / g;
    const int64_t qn = rad_tensor_numel(Q);
    if (qn <= 0 || qn % n) return RAD_E_SHAPE;
    const int64_t M = qn / n;
    if (M > 0xffff) return RAD_E_SHAPE;
    if (rad_tensor_numel(SC) < M * ngrp) return RAD_E_SHAPE;
    if (OB && rad_tensor_numel(OB) < M * n) return RAD_E_SHAPE;

    /* the GEMM over the gate_up plane, with the scratch as its y */
    if (!a->scratch || a->scratch_bytes < M * N * 2 || ((uintptr_t)a->scratch & 15))
        return RAD_E_UNSUPPORTED;
    RadArgs ga = *a;
    RadTensor gt[5];
    for (int i = 0; i < 4; ++i) gt[i] = a->t[i];
    memset(&gt[4], 0, sizeof gt[4]);
    gt[4].data = a->scratch;
    gt[4].dtype = RAD_BF16;
    gt[4].rank = 2;
    gt[4].shape[0] = M;
    gt[4].shape[1] = N;
    gt[4].stride[0] = N;
    gt[4].stride[1] = 1;
    ga.t = gt;
    ga.n_t = 5;
    int64_t gm = 0, gn = 0;
    int rc = entry_preamble(&ga, ENC_FP8A8, 0, &gm, &gn);
    if (rc) return rc;
    rc = plan_fp8a8(&ga, gm, G);
    if (rc) return rc;
    if (G->N != N) return RAD_E_SHAPE;

    int64_t qp = 0, sp = 0, op = 0;
    if (band_row_pitch(Q, n, &qp) || band_row_pitch(SC, ngrp, &sp) ||
        (OB && band_row_pitch(OB, n, &op)))
        return RAD_E_STRIDE;
    E->gu = (const uint8_t*)a->scratch;
    E->q = (uint8_t*)Q->data;
    E->scale = (float*)SC->data;
    E->ob = OB ? (uint8_t*)OB->data : nullptr;
    E->gu_bf16 = 1;
    E->ob_bf16 = OB && OB->dtype == RAD_BF16;
    E->silu = strcmp(act, "sigmoid") != 0;
    E->rows = M;
    E->n = n;
    E->g = g;
    E->ngrp = ngrp;
    E->gu_pitch = N;
    E->q_pitch = qp;
    E->s_pitch = sp;
    E->ob_pitch = op;
    return RAD_OK;
}

bool logits_shape(int64_t M, int64_t K, LogitsShape* out) {
    const int64_t nw = (K + 255) / 256;
    /* Shape: waves a workgroup and windows in flight.  Activation rows are staged
     * nw_pad * 512 + 16 bytes apart, at most 8 rows a pass, and 5..8 rows keep one window
     * in flight (registers); the first shape with LDS for min(M, 8) rows beside the waves'
     * scale tables wins, else the first with room for one row.  R3D_LOGITS_SHAPE="W,D"
     * (W 4|8 waves, D 1..3 windows) is tried first (a tuning lever, read once). */
    const int64_t want = M < 8 ? M : 8;
    static const char* lever = getenv("R3D_LOGITS_SHAPE");
    int shapes[5][2] = {{0, 0}, {8, 2}, {8, 1}, {4, 2}, {4, 1}};
    int lw = 0, ld = 0;
    if (lever && sscanf(lever, "%d,%d", &lw, &ld) == 2 && (lw == 4 || lw == 8) && ld >= 1 && ld <= 3) {
        shapes[0][0] = lw;
        shapes[0][1] = ld;
    }
    for (int pass = 0; pass < 2; ++pass)
        for (const auto& sh : shapes) {
            if (!sh[0]) continue;
            const int np = (int)((nw + sh[1]) / (sh[1] + 1) * (sh[1] + 1));
            const int64_t xr = (int64_t)np * 512 + 16, st = (int64_t)sh[0] * 16 * 2 * np * 4;
            int64_t rows = (kLogitsLds - st) / xr;
            if (rows < 1) continue;
            if (rows > want) rows = want;
            if (rows > 4 && sh[1] > 1) rows = 4;
            /* first pass: a shape that holds the wanted rows (the lever: any that fits) */
            if (pass == 0 && rows < want && &sh != &shapes[0]) continue;
            if (out) {
                out->waves = sh[0];
                out->depth = sh[1];
                out->nw_pad = np;
                out->xrow = xr;
                out->stab = st;
                out->mt = rows;
            }
            return true;
        }
    return false;
}

/* The reference entry's gates, in its order and with its codes (src/r3d_gemm_logits.hip:
 * 149-186), then this build's: the codes plane inside the blob's byte count, 32-bit
 * buffer offsets, and one staged activation row within the compute unit's LDS (n_embd up
 * to 40448).  n_embd a multiple of 16 with 16-byte aligned x rows and codes plane and an
 * element-aligned scale plane takes the fast walk; any other multiple of 4 at any
 * alignment the dword walk (ua). */
int plan_logits_e4m3(const RadArgs* a, const RadPlanesHead* hh, LogitsPlan* P, bool args_only) {
    const RadTensor* X = rad_arg_in(a, 0);
    const RadTensor* W = rad_arg_in(a, 1);
    const RadTensor* Y = rad_arg_in(a, 2);
    if (!X || !W || !Y) return RAD_E_UNSUPPORTED;
    const char* dt = rad_args_gets(a, "dtype");
    if (!dt || strcmp(dt, "bf16") != 0) return RAD_E_UNSUPPORTED;
    if (X->dtype != RAD_BF16 || Y->dtype != RAD_F32) return RAD_E_UNSUPPORTED;
    long long N = 0, K = 0;
    if (!rad_args_geti(a, "n_vocab", &N) || !rad_args_geti(a, "n_embd", &K)) return RAD_E_SHAPE;
    if (N <= 0 || K <= 0) return RAD_E_SHAPE;
    const long long yn = rad_tensor_numel(Y);
    if (yn <= 0 || yn % N) return RAD_E_SHAPE;
    const long long M = yn / N;                        /* never the M parameter */
    if (M > kDimMax || N > kDimMax || K > kDimMax) return RAD_E_SHAPE;
    if (rad_tensor_numel(X) < M * K) return RAD_E_SHAPE;
    if (K & 3) return RAD_E_UNSUPPORTED;
    if (X->rank >= 2 && X->stride[X->rank - 1] != 1) return RAD_E_STRIDE;
    if (Y->rank >= 2 && Y->stride[Y->rank - 1] != 1) return RAD_E_STRIDE;
    const int64_t x_pitch = X->rank >= 2 ? X->stride[X->rank - 2] : K;
    const int64_t y_pitch = Y->rank >= 2 ? Y->stride[Y->rank - 2] : N;
    if (x_pitch < K || y_pitch < N || !pitch_ok(x_pitch) || !pitch_ok(y_pitch)) return RAD_E_STRIDE;
    if (args_only) return RAD_OK;

    const RadPlanesHeader* h = hh ? &hh->h : nullptr;
    if (!h || h->magic != RAD_PLANES_MAGIC || h->n_planes != 2) return RAD_E_DTYPE;
    if (h->transform[0]) return RAD_E_UNSUPPORTED;
    const RadPlanesEntry* ec = nullptr;
    const RadPlanesEntry* es = nullptr;
    const void* pc = rad_planes_find_at(h, W->data, "codes", &ec);
    const void* ps = rad_planes_find_at(h, W->data, "scale", &es);
    if (!pc || !ps || !ec || !es) return RAD_E_DTYPE;
    if (ec->dtype != RAD_F8E4M3 || ec->block[0] != 1 || ec->block[1] != 1 || ec->rows != N ||
        ec->cols != K)
        return RAD_E_SHAPE;
    if (es->dtype != RAD_BF16 && es->dtype != RAD_F16 && es->dtype != RAD_F32)
        return RAD_E_UNSUPPORTED;
    if (es->block[1] != 128 || (es->block[0] != 1 && es->block[0] != 128)) return RAD_E_UNSUPPORTED;
    const int64_t srows = (N + es->block[0] - 1) / es->block[0], scols = (K + 127) / 128;
    if (es->rows != srows || es->cols != scols) return RAD_E_SHAPE;
    if (ec->row_bytes != K) return RAD_E_STRIDE;       /* dense, one byte each */
    /* extents in overflow-checked arithmetic (header fields are untrusted bytes): an
     * extent past int64 is past the blob */
    int64_t s_span = 0, s_end = 0, c_end = 0;
    const bool s_ovf = __builtin_mul_overflow(es->rows, es->row_bytes, &s_span) ||
                       __builtin_add_overflow(es->offset, s_span, &s_end);
    if (s_ovf || h->bytes < s_end) return RAD_E_SHAPE;

    /* gfx950 gates */
    const int64_t ssz = es->dtype == RAD_F32 ? 4 : 2;
    if (es->row_bytes < scols * ssz || es->row_bytes % ssz || es->offset < 0 || ec->offset < 0)
        return RAD_E_STRIDE;
    if (__builtin_add_overflow(ec->offset, N * K, &c_end) || h->bytes < c_end) return RAD_E_SHAPE;
    /* buffer offsets are 32-bit: one wave's rows of codes and the whole scale plane */
    if (64 * K > 0x7FFFFFFFLL || s_span > 0x7FFFFFFFLL) return RAD_E_UNSUPPORTED;
    LogitsShape sh{};
    if (!logits_shape(M, K, &sh)) return RAD_E_UNSUPPORTED;
    if ((M + sh.mt - 1) / sh.mt > 65535) return RAD_E_UNSUPPORTED;   /* passes ride grid.y */
    P->ua = (K % 16) || !aligned16(X->data) || (x_pitch & 7) || !aligned16(pc) ||
            ((uintptr_t)ps % ssz);
    P->X = (const uint16_t*)X->data;
    P->codes = (const uint8_t*)pc;
    P->scale = (const uint8_t*)ps;
    P->Y = (float*)Y->data;
    P->sdt = es->dtype == RAD_BF16 ? 0 : es->dtype == RAD_F16 ? 1 : 2;
    P->br = (int)es->block[0];
    P->mt = (int)sh.mt;
    P->nwin = (int)scols;
    P->nw_pad = sh.nw_pad;
    P->xrow = (int)sh.xrow;
    P->waves = sh.waves;
    P->depth = sh.depth;
    P->M = M; P->N = N; P->K = K;
    P->x_pitch = x_pitch;
    P->s_pitch = es->row_bytes / ssz;
    P->y_pitch = y_pitch;
    P->lds = (int)(sh.mt * sh.xrow + sh.stab);
    LogitsGuard& g = P->guard;
    g.header = (const uint8_t*)W->data;
    g.ic = (int32_t)(ec - rad_planes_entries(h));
    g.is = (int32_t)(es - rad_planes_entries(h));
    g.c_off = ec->offset; g.c_rows = ec->rows; g.c_cols = ec->cols;
    g.s_off = es->offset; g.s_rows = es->rows; g.s_row_bytes = es->row_bytes; g.s_br = es->block[0];
    g.s_dtype = es->dtype; g.pad = 0;
    return RAD_OK;
}

LogitsGeom logits_geom(const LogitsPlan& P, int cus, int per_cu) {
    LogitsGeom g{};
    g.chunks = (P.N + 15) / 16;
    int64_t blocks = (g.chunks + P.waves - 1) / P.waves;
    if (blocks > (int64_t)cus * per_cu) blocks = (int64_t)cus * per_cu;
    g.blocks = (int)blocks;
    g.passes = (P.M + P.mt - 1) / P.mt;
    return g;
}

bool env_no_mxfp4()   { static const bool v = getenv("R3D_NO_MXFP4") != nullptr;   return v; }
bool env_no_fp4_dec() { static const bool v = getenv("R3D_NO_FP4_DEC") != nullptr; return v; }
bool env_no_fp8a8()   { static const bool v = getenv("R3D_NO_FP8A8") != nullptr;   return v; }
bool env_no_fp8_dec() { static const bool v = getenv("R3D_NO_FP8_DEC") != nullptr; return v; }
bool env_debug()      { static const bool v = getenv("R3D_DEBUG_GEMM") != nullptr; return v; }
int64_t env_splitk() {
    static const int64_t v = [] {
        const char* e = getenv("R3D_GFX950_SPLITK");
        return e ? (int64_t)atoll(e) : (int64_t)0;
    }();
    return v;
}
int64_t env_quad_waves() {
    static const int64_t v = [] {
        const char* e = getenv("R3D_GFX950_QWAVES");
        const int64_t w = e ? (int64_t)atoll(e) : 0;
        return w > 0 ? w : (int64_t)0;
    }();
    return v;
}

int env_quad_qpw() {
    static const int v = [] {
        const char* e = getenv("R3D_GFX950_QPW");
        return e && atoi(e) == 2 ? 2 : 1;
    }();
    return v;
}

int env_quad_wv() {
    static const int v = [] {
        const char* e = getenv("R3D_GFX950_QWV");
        const int w = e ? atoi(e) : 0;
        return w == 4 || w == 7 || w == 8 ? w : 0;
    }();
    return v;
}

int64_t env_lines_waves() {
    static const int64_t v = [] {
        const char* e = getenv("R3D_GFX950_LWAVES");
        const int64_t w = e ? (int64_t)atoll(e) : 0;
        return w > 0 ? w : (int64_t)4096;
    }();
    return v;
}

int env_lines_depth() {
    static const int v = [] {
        const char* e = getenv("R3D_GFX950_LD");
        return e ? atoi(e) : 0;
    }();
    return v;
}

int env_lines_tw() {
    static const int v = [] {
        const char* e = getenv("R3D_GFX950_LTW");
        return e ? atoi(e) : 0;
    }();
    return v;
}

int env_quad_depth(int enc) {
    static const int v = [] {
        const char* e = getenv("R3D_GFX950_QD");
        return e ? atoi(e) : 0;
    }();
    (void)enc;
    return v > 0 ? v : 0;   /* 0: the policy in quad_geom */
}

bool decode_fuse(const RadArgs* a) {
    if (a && a->tv)
        for (int i = 0; i < a->n_tv; ++i)
            if (a->tv[i].name && strcmp(a->tv[i].name, "fuse") == 0) return a->tv[i].value > 0;
    return false;
}

int64_t decode_splitk(const RadArgs* a) {
    if (a && a->tv)
        for (int i = 0; i < a->n_tv; ++i)
            if (a->tv[i].name && strcmp(a->tv[i].name, "splitk") == 0 && a->tv[i].value > 0)
                return a->tv[i].value;
    return env_splitk();
}

int describe(const char* row, const RadArgs* a, char* buf, int len) {
    if (!row || !buf || len <= 0) return RAD_E_INVAL;
    if (strstr(row, "quant_act_fp8") != nullptr) {
        QuantPlan Q{};
        const int rc = plan_quant_act_fp8(a, &Q);
        if (rc) { snprintf(buf, (size_t)len, "refused rc=%d (plan)", rc); return rc; }
        snprintf(buf, (size_t)len,
                 "arm=band op=quant_act_fp8 x=%s rows=%lld n=%lld group=%lld ngrp=%lld "
                 "x_pitch=%lld q_pitch=%lld s_pitch=%lld",
                 Q.x_bf16 ? "bf16" : "f32", (long long)Q.rows, (long long)Q.n, (long long)Q.g,
                 (long long)Q.ngrp, (long long)Q.x_pitch, (long long)Q.q_pitch,
                 (long long)Q.s_pitch);
        return RAD_OK;
    }
    if (strstr(row, "logits_gemm") != nullptr) {
        /* describe copies nothing from the device: the blob's header is read in place when
         * it is host-accessible, else taken from the copy an earlier launch cached */
        const RadTensor* W = rad_arg_in(a, 1);
        LogitsPlan L{};
        int rc = plan_logits_e4m3(a, nullptr, &L, true);
        RadPlanesHead hc;
        if (!rc && !logits_head_peek(W->data, &hc)) {
            snprintf(buf, (size_t)len, "refused rc=%d (the blob's header is in device memory "
                     "and no launch has cached it: not host-readable)", RAD_E_UNSUPPORTED);
            return RAD_E_UNSUPPORTED;
        }
        if (!rc) rc = plan_logits_e4m3(a, &hc, &L, false);
        if (rc) { snprintf(buf, (size_t)len, "refused rc=%d (plan)", rc); return rc; }
        const LogitsGeom g = logits_geom(L, 256, 1);
        snprintf(buf, (size_t)len,
                 "arm=logits M=%lld N=%lld K=%lld mt=%d passes=%lld depth=%d wg_waves=%d "
                 "chunks=%lld blocks=%d br=%d sdt=%d nwin=%d lds=%d walk=%s",
                 (long long)L.M, (long long)L.N, (long long)L.K, L.mt, (long long)g.passes,
                 L.depth, L.waves, (long long)g.chunks, g.blocks, L.br, L.sdt, L.nwin, L.lds,
                 L.ua ? "dword" : "vector");
        return RAD_OK;
    }
    if (strstr(row, "rmsnorm_quant_fp8") != nullptr) {
        RmsPlan R{};
        const int rc = plan_rmsnorm_quant_fp8(a, &R);
        if (rc) { snprintf(buf, (size_t)len, "refused rc=%d (plan)", rc); return rc; }
        snprintf(buf, (size_t)len,
                 "arm=band op=rmsnorm_quant_fp8 rows=%lld n=%lld group=%lld ngrp=%lld w=%s "
                 "residual=%d ob=%s eps=%.9g wadd=%.9g x_pitch=%lld q_pitch=%lld s_pitch=%lld",
                 (long long)R.rows, (long long)R.n, (long long)R.g, (long long)R.ngrp,
                 R.w_bf16 ? "bf16" : "f32", R.res != nullptr,
                 R.ob ? (R.ob_bf16 ? "bf16" : "f32") : "none", (double)R.eps, (double)R.wadd,
                 (long long)R.x_pitch, (long long)R.q_pitch, (long long)R.s_pitch);
        return RAD_OK;
    }
    if (strstr(row, "gemm_nt_q_gated") != nullptr) {
        GemmPlan G{};
        GatedPlan E{};
        const int rc = plan_gemm_gated(a, &G, &E);
        if (rc) { snprintf(buf, (size_t)len, "refused rc=%d (plan)", rc); return rc; }
        snprintf(buf, (size_t)len,
                 "arm=gated gemm=%s M=%lld N=%lld K=%lld n=%lld group=%lld act=%s ob=%s rblk=%d",
                 G.M <= 16 && !env_no_fp8_dec() ? "decode" : "prefill", (long long)G.M,
                 (long long)G.N, (long long)G.K, (long long)E.n, (long long)E.g,
                 E.silu ? "silu" : "sigmoid", E.ob ? (E.ob_bf16 ? "bf16" : "f32") : "none",
                 G.rblk);
        return RAD_OK;
    }
    if (strstr(row, "gated_quant_fp8") != nullptr) {
        GatedPlan E{};
        const int rc = plan_gated_quant_fp8(a, &E);
        if (rc) { snprintf(buf, (size_t)len, "refused rc=%d (plan)", rc); return rc; }
        snprintf(buf, (size_t)len,
                 "arm=band op=gated_quant_fp8 gate_up=%s rows=%lld n=%lld group=%lld ngrp=%lld "
                 "act=%s ob=%s gu_pitch=%lld q_pitch=%lld s_pitch=%lld ob_pitch=%lld",
                 E.gu_bf16 ? "bf16" : "f32", (long long)E.rows, (long long)E.n, (long long)E.g,
                 (long long)E.ngrp, E.silu ? "silu" : "sigmoid",
                 E.ob ? (E.ob_bf16 ? "bf16" : "f32") : "none", (long long)E.gu_pitch,
                 (long long)E.q_pitch, (long long)E.s_pitch, (long long)E.ob_pitch);
        return RAD_OK;
    }
    const bool a16 = strstr(row, "mxfp4a16") != nullptr;
    const bool mx = strstr(row, "mxfp4") != nullptr;
    const bool dec = strstr(row, "decode") != nullptr;
    const int enc = a16 ? ENC_MXFP4A16 : mx ? ENC_MXFP4A8 : ENC_FP8A8;
    const char* ename = a16 ? "mxfp4a16" : mx ? "mxfp4a8" : "fp8a8";
    int64_t M = 0, N = 0;
    int rc = entry_preamble(a, enc, dec ? 16 : 0, &M, &N);
    if (rc) { snprintf(buf, (size_t)len, "refused rc=%d (preamble)", rc); return rc; }
    GemmPlan P{};
    rc = a16 ? plan_mxfp4a16(a, M, N, &P) : mx ? plan_mxfp4a8(a, M, N, &P) : plan_fp8a8(a, M, &P);
    if (rc) { snprintf(buf, (size_t)len, "refused rc=%d (plan)", rc); return rc; }
    QuadGeom qg{};
    const bool quad = quad_fits(P) && quad_geom(P.enc, P.M, P.N, P.K, decode_splitk(a), &qg, P.xq);
    auto wide_line = [&](const WideGeom& w, int kc, const char* arm) {
        snprintf(buf, (size_t)len,
                 "arm=%s kernel=wide enc=%s M=%lld N=%lld K=%lld bn=%d tiles=%lld kc=%d "
                 "cst=%d steps=%lld ntg=%d tw=%d depth=%d lds=%d partials=%lld (f32 partial "
                 "planes in scratch, summed in chunk order)",
                 arm, ename, (long long)P.M, (long long)P.N, (long long)P.K, 128 * w.tw,
                 (long long)w.ntiles, kc, w.cg, (long long)(P.K / 128), w.ntg, w.tw, w.d,
                 w.lds, (long long)kc * P.M * P.N * 4);
    };
    int dkc = 0;
    WideGeom dw{};
    if (P.ua & UA_GEMM) {
        snprintf(buf, (size_t)len,
                 "arm=any kernel=any enc=%s M=%lld N=%lld K=%lld tm=%d grid=%lldx%lld rblk=%d "
                 "quant=%s (operands off 16-byte alignment: dword loads, funnel-shifted)",
                 ename, (long long)P.M, (long long)P.N, (long long)P.K, P.M <= 16 ? 1 : 2,
                 (long long)((P.N + 127) / 128),
                 (long long)((P.M + (P.M <= 16 ? 15 : 31)) / (P.M <= 16 ? 16 : 32)), P.rblk,
                 !a16 ? "none" : (P.ua & UA_QUANT) ? "elementwise" : "vector");
        return RAD_OK;
    }
    if (dec && !P.xq && a->scratch && ((uintptr_t)a->scratch & 15) == 0 &&
        decode_split_plan(P.enc, P.M, P.N, P.K, 256, quad, decode_splitk(a), &dkc, &dw) &&
        a->scratch_bytes >= (int64_t)dkc * P.M * P.N * 4) {
        wide_line(dw, dkc, "splitk");
    } else if (dec && quad) {
        snprintf(buf, (size_t)len,
                 "arm=decode kernel=quad enc=%s M=%lld N=%lld K=%lld mt=%d qpw=%d chunks=%d "
                 "waves=%d quads=%lld blocks=%lld groups=%d depth=%d lds=%d rblk=%d xq=%d",
                 ename, (long long)P.M, (long long)P.N, (long long)P.K, qg.mt, qg.qpw, qg.chunks,
                 qg.wv,
                 (long long)qg.quads, (long long)qg.blocks, qg.groups, qg.depth, qg.lds, P.rblk,
                 P.xq);
    } else if (dec && P.xq) {
        snprintf(buf, (size_t)len, "refused rc=%d (fused bf16 activations need the quad GEMV)",
                 RAD_E_UNSUPPORTED);
        return RAD_E_UNSUPPORTED;
    } else if (LinesGeom lg{}; dec && lines_fits(P) &&
               lines_geom(P.enc, P.M, P.N, P.K, decode_splitk(a), &lg)) {
        snprintf(buf, (size_t)len,
                 "arm=decode kernel=lines enc=%s M=%lld N=%lld K=%lld mt=%d tw=%d chunks=%d waves=4 "
                 "tiles=%lld blocks=%lld units=%d depth=%d lds=%d rblk=%d",
                 ename, (long long)P.M, (long long)P.N, (long long)P.K, lg.mt, lg.tw, lg.chunks,
                 (long long)lg.tiles, (long long)lg.blocks, lg.units, lg.depth, lg.lds, P.rblk);
    } else if (dec) {
        DecodeGeom g{};
        decode_geom(P.M, P.N, P.K, decode_splitk(a), &g,
                    gemv_wave_lds(P.enc, P.M <= 1 ? 1 : P.M <= 4 ? 4 : 16));
        snprintf(buf, (size_t)len,
                 "arm=decode kernel=tile16 enc=%s M=%lld N=%lld K=%lld mt=%d chunks=%d waves=%d tiles=%lld "
                 "blocks=%lld steps=%d rblk=%d",
                 ename, (long long)P.M, (long long)P.N, (long long)P.K,
                 g.mt, g.chunks, g.waves, (long long)g.tiles, (long long)g.blocks, g.steps,
                 P.rblk);
    } else if (int kc = 0, cst = 0, kind = a->scratch && ((uintptr_t)a->scratch & 15) == 0
                                  ? splitk_plan(P.enc, P.M, P.N, P.K, 256, &kc, &cst, nullptr,
                                                nullptr) : 0;
               kind && a->scratch_bytes >= (int64_t)kc * P.M * P.N * 4) {
        PrefillGeom g{};
        WideGeom w{};
        splitk_plan(P.enc, P.M, P.N, P.K, 256, nullptr, nullptr, &g, &w);
        if (kind == 1)
            wide_line(w, kc, "splitk");
        else
            snprintf(buf, (size_t)len,
                     "arm=splitk kernel=tile enc=%s M=%lld N=%lld K=%lld bn=%d bm=%d tiles=%lld "
                     "kc=%d cst=%d steps=%d lds=%d partials=%lld (f32 partial planes in scratch, "
                     "summed in chunk order)",
                     ename, (long long)P.M, (long long)P.N, (long long)P.K, g.bn, g.bm,
                     (long long)g.tiles, kc, cst, g.steps, g.lds, (long long)kc * P.M * P.N * 4);
    } else if (const int passes = skinny_passes(P.enc, P.M, P.N, 256)) {
        snprintf(buf, (size_t)len,
                 "arm=skinny enc=%s M=%lld N=%lld K=%lld passes=%d (16-row decode GEMV passes)",
                 ename, (long long)P.M, (long long)P.N, (long long)P.K, passes);
    } else {
        const int mode = a16 ? PF_MX8 : mx ? PF_A8 : PF_F8;
        PrefillGeom g{};
        prefill_geom(P.M, P.N, P.K, mode, 256, &g);
        snprintf(buf, (size_t)len,
                 "arm=prefill enc=%s M=%lld N=%lld K=%lld bn=%d bm=%d waves=%d grid=%lldx%lld "
                 "tiles=%lld nst=%d lds=%d steps=%d rblk=%d nsplit=%lld quant=%s",
                 ename, (long long)P.M, (long long)P.N, (long long)P.K, g.bn, g.bm, g.wv,
                 (long long)g.grid_n, (long long)g.grid_m, (long long)g.tiles, g.nst, g.lds,
                 g.steps, P.rblk,
                 (long long)(mode == PF_F8 && g.wv == 4 ? prefill_f8_split_n(P.M, P.N, 256) : 0),
                 !a16 ? "none" : (P.ua & UA_QUANT) ? "elementwise" : "vector");
    }
    return RAD_OK;
}

}  // namespace r3d
