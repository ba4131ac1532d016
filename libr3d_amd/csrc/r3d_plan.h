/* r3d_plan.h -- host-side plans for the gfx950 gemm_nt_q rows: the format / shape /
 * stride gates every entry runs before it launches, and the launch geometry it picks.
 * Pure host C++ (no HIP), so every refusal and every geometry choice is testable on a
 * machine without a GPU.
 */
#ifndef R3D_PLAN_H
#define R3D_PLAN_H

#include <stdint.h>
#include "rad_abi.h"
#include "rad_planes.h"

namespace r3d {

/* ENC_MXFP4A16: e2m1 weights as mxfp4a8, bf16 activations quantised by the library to
 * mxfp8 (e4m3 + E8M0 per 32 of K) in launch scratch before the prefill GEMM. */
enum Encoding { ENC_MXFP4A8 = 0, ENC_FP8A8 = 1, ENC_MXFP4A16 = 2 };

struct GemmPlan {
    int enc;
    const uint8_t* A;        /* e4m3 [M, K] (mxfp4a16: bf16 [M, K]) */
    const float*   AS;       /* f32 [M, K/128] (mxfp4a16: none) */
    const uint8_t* B;        /* mxfp4: [N, K/2] packed e2m1; fp8a8: [N, K] e4m3 */
    const void*    BS;       /* mxfp4: E8M0 [N, K/32]; fp8a8: bf16 [N or N/128, K/128] */
    uint16_t*      Y;        /* bf16 [M, N] */
    int64_t M, N, K;
    int64_t a_pitch, as_pitch, b_pitch, bs_pitch, y_pitch;   /* bytes for A/B, elements else
                                                                (mxfp4a16 A: elements) */
    int as_cols, bs_cols;
    int rblk;                /* fp8a8 weight-scale rows per scale row: 1 or 128 */
    int xq;                  /* decode rows at M = 1 (M <= 4 with the "fuse" tunable): A is
                                bf16 rows (a_pitch bytes), AS absent -- quantised in the
                                kernel with quant_act_fp8's arithmetic */
    uint8_t* scratch;        /* mxfp4a16: e4m3 codes [M, K] then E8M0 [M, K/32] */
    int ua;                  /* operands off the fast arms' alignment: UA_GEMM -- A, B or a
                                scale plane (the any-alignment GEMM, r3d_gemm_any.h, takes the
                                launch); UA_QUANT -- mxfp4a16's bf16 A (its quantiser reads it
                                element by element) */
};
enum { UA_GEMM = 1, UA_QUANT = 2 };

/* Launch scratch the mxfp4a16 row needs at M rows: the e4m3 plane (rounded up to 256
 * bytes) followed by the E8M0 plane. */
int64_t mxfp4a16_scratch_bytes(int64_t M, int64_t K);

/* Which kernel family an entry launches. */
enum Arm { ARM_DECODE = 0, ARM_TILE = 1 };

/* Launch geometry of the decode GEMV: a 16-row weight tile per wave, the K steps (128
 * wide) of a tile split over `chunks` waves of the same workgroup, reduced through LDS
 * in chunk order. */
struct DecodeGeom {
    int mt;                  /* activation rows the kernel instantiation covers: 1, 4, 16 */
    int chunks;              /* waves per tile (split-K), 1/2/4/8 */
    int waves;               /* waves per workgroup */
    int tiles_per_block;
    int64_t tiles;           /* ceil(N / 16) */
    int64_t blocks;
    int steps;               /* K / 128 */
};

/* Launch geometry of the quad decode GEMV (M <= 4): one wave per block of qpw quads (4
 * weight rows each) and K chunk, 4 waves per workgroup (4 / chunks blocks x chunks). */
struct QuadGeom {
    int mt;                  /* activation rows of the instantiation: 1 or 4 */
    int qpw;                 /* quads per wave: 1 or 2 */
    int wv;                  /* waves per workgroup: 4 or 8 */
    int chunks;              /* waves per row block (split-K): 1, 2 or 4 */
    int bpb;                 /* row blocks per workgroup: wv / chunks */
    int groups;              /* K / 128 */
    int gmax;                /* most groups one chunk holds: ceil(groups / chunks) */
    int depth;               /* ring depth in K steps (<= every wave's step count) */
    int64_t quads, nblk, blocks;   /* ceil(N/4); row blocks of 4 qpw rows; workgroups */
    int xs_off;              /* LDS: activation rows at 0 ([mt][K + 16], 1 KB rounded),
                                a_scales ([mt][groups] f32) at xs_off */
    int sc_off, sc_bytes;    /* LDS: weight scales (mxfp4a8: per workgroup; fp8a8: per wave) */
    int lds;                 /* dynamic LDS bytes per workgroup */
};

/* The quad GEMV's LDS layout, computed the same way by the kernel (from K and the chunk
 * count) and by quad_geom: the activation rows [mt][K + 16] bytes at 0, rounded up to 1 KB;
 * the a_scales [mt][groups] f32 at xs_off, rounded up to 256 B; the weight scales at sc_off
 * -- mxfp4a8: the workgroup's rows over the whole K ([rows][groups dwords], rounded up to
 * 1 KB: sc_bytes in all), fp8a8: sc_bytes per wave ([ceil(groups / chunks)][4 qpw rows]
 * 4-byte slots, rounded up to 256 B); the fold after the K loop reuses the start
 * (wv * qpw * 256 bytes).  chunks is a power of two (1, 2 or 4).  A constexpr function,
 * so the kernel's copy is the same code. */
struct QuadLds {
    int64_t xs_off, sc_off, sc_bytes, lds;
};
constexpr QuadLds quad_lds(int enc, int mt, int qpw, int wv, int64_t K, int chunks) {
    const int64_t groups = K >> 7;
    const int64_t blob = ((mt * (K + 16) + 1023) >> 10) << 10;
    const int64_t xs = ((mt * groups * 4 + 255) >> 8) << 8;
    const int cl = __builtin_ctz((unsigned)chunks);
    const int64_t gmax = (groups + chunks - 1) >> cl;
    const int64_t scb = enc == ENC_MXFP4A8
                            ? ((4 * qpw * (int64_t)(wv >> cl) * 4 * groups + 1023) >> 10) << 10
                            : ((16 * qpw * gmax + 255) >> 8) << 8;
    const int64_t lds = blob + xs + (enc == ENC_MXFP4A8 ? scb : wv * scb);
    const int64_t fold = (int64_t)wv * qpw * 256;
    return QuadLds{blob, blob + xs, scb, lds < fold ? fold : lds};
}

/* The line GEMV's per-wave LDS slice (a_scales [16][gmax] f32, then the weight scales of
 * its 16 tw rows over gmax groups, each rounded up to 256 B) for `chunks` (1, 2 or 4) K
 * chunks; the kernel computes it the same way. */
constexpr int lines_wlds(int enc, int tw, int64_t K, int chunks) {
    const int G = enc == ENC_MXFP4A8 ? 2 : 1;
    const int units = (int)(((K >> 7) + G - 1) / G);
    const int gm = G * ((units + chunks - 1) >> __builtin_ctz((unsigned)chunks));
    return (((64 * gm + 255) >> 8) << 8) + (((64 * tw * gm + 255) >> 8) << 8);
}

/* Launch geometry of the line GEMV (M <= 16): one wave per block of tw 16-row weight tiles
 * and K chunk, 4 waves per workgroup (4 / chunks blocks x chunks); a unit is one 128-byte
 * line of every row of the block (2 K groups at mxfp4a8, 1 at fp8a8). */
struct LinesGeom {
    int mt;                  /* activation rows of the instantiation: 8 or 16 */
    int tw;                  /* 16-row tiles per wave: 1, 2 or 4 */
    int chunks;              /* waves per row block (split-K): 1, 2 or 4 */
    int tpb;                 /* row blocks (16 tw rows) per workgroup: 4 / chunks */
    int groups, units;       /* K / 128; lines per row */
    int gmax;                /* most K groups one chunk holds */
    int depth;               /* ring depth in units (<= every wave's unit count) */
    int wlds;                /* LDS bytes of one wave's scale tables */
    int lds;                 /* dynamic LDS bytes per workgroup */
    int64_t tiles, nblk, blocks;   /* ceil(N/16); row blocks of 16 tw rows; workgroups */
};

/* Launch geometry of the prefill GEMM (block-scaled MFMA, direct-to-LDS ring):
 * a workgroup of 8 waves (2 x 4) owns bn = 32 wnf weight rows x bm = 64 wmf tokens. */
struct PrefillGeom {
    int wnf, wmf, nst;       /* 16-row fragments per wave along N / M; ring depth */
    int wv;                  /* waves per workgroup: 8, or 4 (one a SIMD) */
    int bn, bm;
    int64_t grid_m, grid_n, tiles;
    int steps;               /* K / 128 */
    int lds;                 /* dynamic LDS bytes per workgroup */
};

int64_t grid_block(int64_t ext, int64_t blocks);
int64_t row_stride(const RadTensor* t, int64_t cols);

/* Format gates (src/r3d_gemm_mxfp4.hip:1521-1582 and src/r3d_gemm_fp8a8.hip:852-924)
 * plus this build's gfx950 gate K % 128 == 0.  Operands off the fast arms' alignment
 * (16-byte A/B bases and pitches, 4-byte mxfp4 / 2-byte fp8 scale planes, 4-byte
 * a_scale) set ua = UA_GEMM: the any-alignment arm.  M must already be numel(Y)/N.
 * Returns RAD_OK or the refusal code. */
int plan_mxfp4a8(const RadArgs* a, int64_t M, int64_t N, GemmPlan* P);
int plan_fp8a8(const RadArgs* a, int64_t M, GemmPlan* P);
/* The bf16-in mxfp4 row: A bf16 [M, K], a_scale absent, weights as mxfp4a8, and launch
 * scratch of at least mxfp4a16_scratch_bytes(M, K), 16-byte aligned. */
int plan_mxfp4a16(const RadArgs* a, int64_t M, int64_t N, GemmPlan* P);

/* The shared entry preamble: operands present (a_scale except at mxfp4a16, and at the
 * decode rows when `a` is bf16: the fused producer), a_sum (and for fp8a8 b_ref) refused, Y
 * bf16 and inner-contiguous, N from the schema parameter, M = numel(Y)/N (never the M
 * parameter), and the band's own M bound when `m_max` > 0 (a decode row). */
int entry_preamble(const RadArgs* a, int enc, int64_t m_max, int64_t* M, int64_t* N);

/* wave_lds: LDS bytes one wave needs (0 = unknown: assume it fits 8 waves per workgroup). */
void decode_geom(int64_t M, int64_t N, int64_t K, int64_t force_chunks, DecodeGeom* g,
                 int wave_lds = 0);
/* Quad GEMV geometry; false when the shape is outside what it serves (M > 4, or the
 * workgroup's LDS -- whole-K activation rows -- over kQuadMaxLds), and the 16-row GEMV
 * runs instead.  force_chunks: 1/2/4 pin the split, anything else above 0
 * leaves the quad kernel. */
constexpr int kQuadMaxLds = 48 * 1024;
bool quad_geom(int enc, int64_t M, int64_t N, int64_t K, int64_t force_chunks, QuadGeom* g,
               int xq = 0);
/* The quad kernel addresses a wave's (up to 8) weight rows through one buffer resource:
 * they must span less than 2^31 bytes; it takes the operand pitches as 32-bit arguments. */
bool quad_fits(const GemmPlan& P);
/* Line GEMV geometry; false when the shape is outside what it serves (M outside 5..16, or a
 * wave's scale tables over the LDS budget), and the 16-row GEMV runs instead.  force_chunks:
 * 1/2/4 pin the split, anything else above 0 leaves the line kernel. */
constexpr int kLinesMaxLds = 48 * 1024;
bool lines_geom(int enc, int64_t M, int64_t N, int64_t K, int64_t force_chunks, LinesGeom* g);
/* The line kernel addresses a wave's (up to 64) weight rows and the whole activation plane through
 * buffer resources: both must span less than 2^31 bytes. */
bool lines_fits(const GemmPlan& P);
/* mode: PF_A8 = e4m3 activations with f32 scale per 128 (mxfp4a8), PF_MX8 = mxfp8
 * (mxfp4a16), PF_F8 = e4m3 activations and e4m3 weights with bf16 row scales (fp8a8);
 * ncu: compute units the launch can fill (tiles are sized so the last round of
 * workgroups is as full as possible). */
void prefill_geom(int64_t M, int64_t N, int64_t K, int mode, int ncu, PrefillGeom* g);

/* The skinny band (M = 17..64) on the tile rows: the number of 16-row passes of the decode
 * GEMVs to run instead of the prefill pipeline, or 0.  The prefill tile spans 128 weight
 * rows, so a narrow N leaves most CUs idle on a weight-bound problem (~12.5 GB/s per active
 * tile, measured), while the line GEMV runs the passes side by side in one launch (the
 * repeated weight reads mostly hit the caches): passes win while
 * passes x min(tiles, CUs) < 300 (measured on MI355X at config 2's shapes).
 * R3D_GFX950_SKINNY=0 / 1 turns the passes off / on for every skinny shape. */
int skinny_passes(int enc, int64_t M, int64_t N, int ncu);

/* The e4m3 prefill on its four-wave 128 x 256 tile when the tile count leaves the last round
 * part full: weight rows [0, n1) run as whole rounds of that tile and [n1, N) as a second
 * launch on the 128 x 128 tile, where that costs less (a round of the four-wave tile counts
 * 1.71 rounds of the other).  Returns n1 (a multiple of 128), or 0 for one launch over N. */
int64_t prefill_f8_split_n(int64_t M, int64_t N, int ncu);

/* The skinny-band GEMV (gemv_wide_kernel, r3d_gemv_wide.h): 8 waves of tw 16-row weight
 * tiles (256 rows a workgroup at tw = 2) x one K chunk of cg groups; depth d lines in each
 * wave's register ring (1: measured at least as fast as 2 and 4 on every config 2 shape at
 * M = 4..64, and 10 % faster at M = 64); ntg 16-row groups of activations staged in LDS with
 * the chunk. */
struct WideGeom {
    int tw, d;
    int cg, ntg, sclds, lds;
    int64_t ntiles;
};
constexpr int kWideMaxLds = 152 * 1024;

/* Split K on the tile rows (mxfp4a8, fp8a8) up to M = 128, where a narrow N leaves most
 * CUs idle under the prefill pipeline's one tile per 128 weight rows: the K steps are cut
 * into kc chunks of *cst steps (every chunk non-empty), the tile x chunk units write f32
 * partial tiles into the launch scratch and a second kernel sums the chunks in order into
 * bf16 Y.  The split's tile (*g): up to M = 64 one 64-token group a wave (e2m1 weights: 256
 * rows, e4m3: 128), else the 128 x 128 tile.  Returns kc (0: no split).  Units aim at one
 * per CU (R3D_GFX950_SPLITK_UNITS overrides the target, 0 turns the split off) with at
 * least kSplitMinSteps steps a chunk. */
constexpr int kSplitMinSteps = 4;
int tile_splitk(int enc, int64_t M, int64_t N, int64_t K, int ncu, int* cst, PrefillGeom* g);
/* The split's kernel: up to M = 64 the skinny-band GEMV (kind 1, *w), else the 128 x 128
 * prefill tile (kind 2, *g); 0 when no split applies.  *kc and *cst as tile_splitk's.
 * R3D_GFX950_SPLITK_KERNEL=tile keeps the prefill tile (64 tokens a tile) up to M = 64. */
int splitk_plan(int enc, int64_t M, int64_t N, int64_t K, int ncu, int* kc, int* cst,
                PrefillGeom* g, WideGeom* w);
/* Launch scratch the split needs: kc f32 planes of M x N (0 without a split). */
int64_t tile_splitk_bytes(int enc, int64_t M, int64_t N, int64_t K, int ncu);
/* The tile rows' scratch hook: tile_splitk_bytes at the args' N and K and M (numel(y) / N,
 * else the "M" param, else 128 -- the largest M the split takes); 0 without N or K. */
int64_t tile_scratch_bytes(const RadArgs* a, int enc, int ncu);

/* The decode rows' K split over launch scratch: the skinny-band GEMV's split (splitk_plan
 * kind 1) takes the launch where the decode arm would be the line GEMV (M = 5..16) or the
 * 16-row GEMV (an M <= 4 shape the quad GEMV cannot stage), on a plane of at least
 * kDecodeSplitMinWeights weights and with no pinned split (pin > 0: the row's "splitk"
 * tunable).  Measured on MI355X at config 2's shapes: gate_up / down M = 16 20.7 / 25.9 us
 * on the line GEMV, 16.9 / 16.7 us split; qkv (N K = 44 M) is faster unsplit at every M.
 * quad: the quad GEMV takes this launch.  Returns 1 with *kc chunks of geometry *w, else 0. */
constexpr int64_t kDecodeSplitMinWeights = (int64_t)1 << 26;
int decode_split_plan(int enc, int64_t M, int64_t N, int64_t K, int ncu, bool quad, int64_t pin,
                      int* kc, WideGeom* w);
/* The decode rows' scratch hook: the split's kc f32 planes of M x N at the args' N, K and M
 * (numel(y) / N, else the "M" param, else 16), 0 where the split does not apply. */
int64_t decode_scratch_bytes(const RadArgs* a, int enc, int ncu);

/* The band rows' operand walk (src/r3d_band.hip:419-449 of the reference): a rank-1 tensor
 * of exactly `cols` unit-stride elements is one row read by every row (pitch 0); rank 2
 * needs a unit inner stride and pitches by stride[0] when shape[1] == cols, else reads flat
 * (pitch cols); rank >= 3 needs a unit inner stride and, when the last extent is cols,
 * contiguous leading dimensions (pitch cols).  Returns 0 and sets *pitch (elements), or a
 * negative code for a layout the walk refuses. */
int band_row_pitch(const RadTensor* t, int64_t cols, int64_t* pitch);

/* quant_act_fp8 launch plan (src/r3d_band.hip:460-487): operands x (f32 or bf16), q (e4m3),
 * scale (f32); n from the param (default x's second extent), rows = numel(x) / n (at most
 * 65535), group from the param clamped to [1, n] (absent or out of range: n).  Returns
 * RAD_OK or the reference's refusal code. */
struct QuantPlan {
    const uint8_t* x;
    uint8_t* q;
    float* scale;
    int x_bf16;
    int64_t rows, n, g, ngrp;
    int64_t x_pitch, q_pitch, s_pitch;        /* elements */
};
int plan_quant_act_fp8(const RadArgs* a, QuantPlan* P);

/* gated_quant_fp8 launch plan (src/r3d_band.hip:492-541): gate_up (f32 or bf16, [rows, 2n]:
 * gate columns [0, n), up columns [n, 2n)), q (e4m3), scale (f32), optional out_bf16 (f32
 * or bf16); n from the param (default half of gate_up's second extent); act "sigmoid"
 * selects sigmoid(gate) * up, anything else (or absent) silu(gate) * up; group as
 * quant_act_fp8's.  Returns RAD_OK or the reference's refusal code. */
struct GatedPlan {
    const uint8_t* gu;
    uint8_t* q;
    float* scale;
    uint8_t* ob;                              /* null: no gated output */
    int gu_bf16, ob_bf16, silu;
    int64_t rows, n, g, ngrp;
    int64_t gu_pitch, q_pitch, s_pitch, ob_pitch;   /* elements */
};
int plan_gated_quant_fp8(const RadArgs* a, GatedPlan* P);

/* rmsnorm_quant_fp8 launch plan (src/r3d_more.hip:482-521): x (bf16), optional residual
 * (bf16, updated in place: the fused add form), w (f32 or bf16, rank 1), q (e4m3), scale
 * (f32), optional out_bf16 (f32 or bf16); n from the param (default w's extent, at most
 * 30720: the row is staged in LDS), group clamped to [1, n] (absent: n), eps (F64, default
 * 1e-6) and wadd (F64, default 0) narrowed to f32.  Returns RAD_OK or the reference's
 * refusal code. */
struct RmsPlan {
    const uint8_t* x;
    uint8_t* res;                             /* null: no residual */
    const uint8_t* w;
    uint8_t* q;
    float* scale;
    uint8_t* ob;                              /* null: no normed output */
    int w_bf16, ob_bf16;
    int64_t rows, n, g, ngrp;
    int64_t x_pitch, r_pitch, q_pitch, s_pitch, ob_pitch;   /* elements */
    float eps, wadd;
};
int plan_rmsnorm_quant_fp8(const RadArgs* a, RmsPlan* P);

/* gemm_nt_q_gated at fp8a8 (src/r3d_gemm_fp8a8.hip:1166-1241): operands a, a_scale, b,
 * b_scale, q, scale, out_bf16?, a_sum? (refused); params N (= 2n, even), K, group, dtype,
 * act (required: silu or sigmoid).  M = numel(q) / n.  The GEMM writes the [M, N] bf16
 * gate_up plane into the launch scratch (at least M*N*2 bytes, 16-byte aligned, else
 * RAD_E_UNSUPPORTED) -- G is the fp8a8 plan for that plane -- and E is gated_quant_fp8's
 * plan over it.  Returns RAD_OK or the reference's refusal code. */
int plan_gemm_gated(const RadArgs* a, GemmPlan* G, GatedPlan* E);
int64_t gemm_gated_scratch_bytes(const RadArgs* a);   /* 64 * N * 2, or 0 without N */

/* logits_gemm over a joined e4m3 + block-scale head (src/r3d_gemm_logits.hip:149-186):
 * x bf16 [M, K] (K = n_embd), lm_head a joined-planes blob (rad_planes.h) holding "codes"
 * (e4m3 [N, K] dense) and "scale" (bf16 / f16 / f32, one per (1 or 128 rows, 128 cols)),
 * logits f32 [M, N] (N = n_vocab); M = numel(logits) / N.  The plane addresses are the
 * blob's (W->data) plus the header's offsets; `guard` carries what the kernel re-checks
 * against the device copy of the header before it reads a plane. */
struct LogitsGuard {
    const uint8_t* header;   /* the blob's first byte (its header, then its entries) */
    int32_t ic, is;          /* entry indices of "codes" and "scale" */
    int64_t c_off, c_rows, c_cols;
    int64_t s_off, s_rows, s_row_bytes, s_br;
    uint32_t s_dtype, pad;
};
struct LogitsPlan {
    const uint16_t* X;
    const uint8_t* codes;
    const uint8_t* scale;
    float* Y;
    int sdt;                 /* scale element: 0 bf16, 1 f16, 2 f32 */
    int br;                  /* weight rows per scale row: 1 or 128 */
    int mt;                  /* activation rows per pass (1..8); passes = ceil(M / mt) */
    int nwin;                /* 128-wide scale blocks along K */
    int nw_pad;              /* 256-wide code windows, padded to the ring's unroll */
    int xrow;                /* LDS pitch of one staged activation row, bytes */
    int waves, depth;        /* waves a workgroup; windows in flight per wave (1..3) */
    int64_t M, N, K;
    int64_t x_pitch, s_pitch, y_pitch;   /* elements */
    int lds;                 /* dynamic LDS bytes per workgroup: x rows, then scale tables */
    int ua;                  /* n_embd off a multiple of 16, or x / codes / scale off the fast
                                walk's alignment: every piece read by dwords, funnel-shifted */
    LogitsGuard guard;
};
/* `h` null: the gates that need no header (args_only); else a host copy of the blob's
 * header and entries. */
int plan_logits_e4m3(const RadArgs* a, const RadPlanesHead* h, LogitsPlan* P, bool args_only);
/* The kernel's shape for M activation rows of n_embd K: waves a workgroup, windows in
 * flight, padded windows, LDS row pitch, scale-table bytes and rows a pass; false when no
 * shape stages even one activation row (K too long for the compute unit's LDS). */
struct LogitsShape {
    int waves, depth, nw_pad;
    int64_t xrow, stab, mt;
};
bool logits_shape(int64_t M, int64_t K, LogitsShape* s);
/* The header (and entries) of the blob at `blob` without copying from device memory: read
 * in place when the blob is host-accessible, else this device's cached copy from an
 * earlier launch; false when neither exists. */
bool logits_head_peek(const void* blob, RadPlanesHead* out);
constexpr int kLogitsLds = 160 * 1024;         /* LDS of one compute unit */
/* The grid: 16-row chunks dealt to waves blocks * waves apart, at most per_cu workgroups
 * per compute unit (what one unit holds at once); blocks.y = passes over the activation
 * rows. */
struct LogitsGeom {
    int64_t chunks;
    int blocks;
    int64_t passes;
};
LogitsGeom logits_geom(const LogitsPlan& P, int cus, int per_cu);

/* The current device: gfx950 or not (answered once per device), and its compute units. */
bool chip_ok();
int cu_count();

/* Environment levers, read once per process (function-local statics). */
bool env_no_mxfp4();        /* R3D_NO_MXFP4: all mxfp4a8 rows */
bool env_no_fp4_dec();      /* R3D_NO_FP4_DEC: the mxfp4a8 decode row */
bool env_no_fp8a8();        /* R3D_NO_FP8A8: all fp8a8 rows */
bool env_no_fp8_dec();      /* R3D_NO_FP8_DEC: the fp8a8 decode row */
bool env_debug();           /* R3D_DEBUG_GEMM: one stderr line per distinct launch arm */
int64_t env_splitk();       /* R3D_GFX950_SPLITK: force the decode chunk count (0 = policy) */
int64_t env_quad_waves();   /* R3D_GFX950_QWAVES: waves the quad split aims for (0: unset) */
int env_quad_depth(int enc);/* R3D_GFX950_QD: quad ring depth 1/2/4/8 (0: unset, the policy) */
int env_quad_qpw();         /* R3D_GFX950_QPW: quads per wave of the quad GEMV, 1 or 2 (default 1) */
int env_quad_wv();          /* R3D_GFX950_QWV: waves per quad-GEMV workgroup, 4 or 8 (0: policy) */
int64_t env_lines_waves();  /* R3D_GFX950_LWAVES: waves the line GEMV's split aims for (default 4096) */
int env_lines_depth();      /* R3D_GFX950_LD: line GEMV ring depth in units, 1/2/4 (0 = policy) */
int env_lines_tw();         /* R3D_GFX950_LTW: 16-row tiles per wave of the line GEMV (0 = policy) */

/* The decode rows' "splitk" tunable (RadArgs::tv): chunks per tile, 0 = the policy.  An
 * engine-chosen value wins over R3D_GFX950_SPLITK. */
int64_t decode_splitk(const RadArgs* a);
/* The decode rows' "fuse" tunable: 1 lets a bf16 activation call at M = 2..4 quantise
 * inside the quad GEMV (default 0: only M = 1 is fused; the engine runs the producer). */
bool decode_fuse(const RadArgs* a);

/* Human-readable plan + geometry for `row` without launching anything. */
int describe(const char* row, const RadArgs* a, char* buf, int len);

}  // namespace r3d

#endif /* R3D_PLAN_H */
