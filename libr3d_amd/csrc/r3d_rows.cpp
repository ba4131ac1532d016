/* r3d_rows.cpp -- plugin identity, the op schemas and the gfx950 row table of
 * libr3d_gfx950, behind radiance's kernel-plugin ABI 26 (src/r3d_rows.cpp:14-27,
 * 2238-2278 of the reference).  Pure host C++.
 *
 * Rows (resolver: per op and band, the highest-priority row whose constraints hold;
 * src/r3d_rows.cpp:1165-1177):
 *   gemm_nt_q_mxfp4          prio 1000  dtype IN mxfp4a8, K DIV 128      prefill GEMM
 *   gemm_nt_q_mxfp4_decode   prio 1100  + M LE 16                         decode GEMV
 *   gemm_nt_q_fp8a8          prio 1000  dtype IN fp8a8, K DIV 128, group EQ 128
 *   gemm_nt_q_fp8a8_decode   prio 1100  + M LE 16
 *   gemm_nt_q_mxfp4a16       prio 1000  dtype IN mxfp4a16, K DIV 128     bf16-in prefill
 *   quant_act_fp8_act        prio 1000  n GE 1, dtype IN f32 bf16          activation producer
 *   gated_quant_fp8_act      prio 1000  n GE 1, dtype IN f32 bf16          gated producer
 *   rmsnorm_quant_fp8        prio 1000  n DIV 4, group EQ 128, dtype IN bf16  norm producer
 *   gemm_nt_q_gated_fp8a8    prio 1000  dtype IN fp8a8, M LE 64, K DIV 128, group EQ 128,
 *                                       act IN silu sigmoid              GEMM + gated producer
 *   logits_gemm_e4m3         prio 1000  n_vocab GE 1, n_embd GE 128, dtype IN bf16
 *                                                                         joined e4m3 lm_head
 * gemm_nt_q_mxfp4a16 has no counterpart in the reference: it takes bf16 activations (no
 * a_scale), quantises them to mxfp8 (e4m3 + E8M0 per 32 of K) in the launch scratch its
 * hook sizes, and runs the prefill GEMM with both block scales inside the MFMA.
 * Deviations from the reference rows (src/r3d_rows.cpp:1601-1675): the decode bands
 * widen M <= 8 to M <= 16 (one MFMA covers 16 activation rows at the cost of one), and
 * the mxfp4 tile row adds K DIV 128 (the MFMA walks whole 128-wide steps; ragged K
 * resolves past the row, to the host reference, as the reference's fp8 row already does).
 *
 * Kill switches act HERE, at registration (src/r3d_rows.cpp:2197-2236): an issue-time
 * refusal is an engine abort, so a lever hides rows and the band re-resolves.
 *   R3D_NO_MXFP4   hides every mxfp4 row;    R3D_NO_FP4_DEC  the mxfp4a8 decode row;
 *   R3D_NO_FP8A8   hides the fp8a8 rows (and the gated row); R3D_NO_FP8_DEC  the fp8a8
 *                  decode row (the gated row then runs its GEMM on the prefill pipeline).
 * Presence-tested (getenv != null), read once.  R3D_MXFP4_Q8X is accepted and inert:
 * this library has no repacked-plane arm for it to withdraw.
 */
#include <stdint.h>
#include <string.h>

#include "rad_abi.h"
#include "r3d_plan.h"

extern "C" {
int r3d_rad_gemm_nt_q(const RadArgs* a, RadStream s);
int r3d_rad_gemm_nt_q_mxfp4_decode(const RadArgs* a, RadStream s);
int r3d_rad_gemm_nt_q_fp8(const RadArgs* a, RadStream s);
int r3d_rad_gemm_nt_q_fp8_decode(const RadArgs* a, RadStream s);
int64_t r3d_rad_gemm_nt_q_scratch(const RadArgs* a);
int64_t r3d_rad_gemm_nt_q_fp8_scratch(const RadArgs* a);
int64_t r3d_rad_gemm_nt_q_mxfp4_decode_scratch(const RadArgs* a);
int64_t r3d_rad_gemm_nt_q_fp8_decode_scratch(const RadArgs* a);
int r3d_rad_gemm_nt_q_mxfp4a16(const RadArgs* a, RadStream s);
int64_t r3d_rad_gemm_nt_q_mxfp4a16_scratch(const RadArgs* a);
int r3d_rad_quant_act_fp8(const RadArgs* a, RadStream s);
int r3d_rad_gated_quant_fp8(const RadArgs* a, RadStream s);
int r3d_rad_rmsnorm_quant_fp8(const RadArgs* a, RadStream s);
int r3d_rad_gemm_nt_q_gated_fp8(const RadArgs* a, RadStream s);
int64_t r3d_rad_gemm_nt_q_gated_fp8_scratch(const RadArgs* a);
int r3d_rad_logits_gemm_e4m3(const RadArgs* a, RadStream s);
int r3d_layout_head(const RadParam*, int, int, const RadEncoding*, const int*, const RadTensor*,
                    int, RadLayout*);
int r3d_relayout_head(const RadParam*, int, int, const RadEncoding*, const int*,
                      const RadTensor*, int, void*, int64_t);
int r3d_unrelayout_head(const RadParam*, int, int, const RadEncoding*, const int*, const void*,
                        int64_t, const RadTensor*, int);
}

namespace {

/* gemm_nt_q's schema: parameter and operand lists exactly as the reference declares
 * them (src/r3d_rows.cpp:186-210), so a loader's schema comparison passes when this
 * library co-loads with another declarer of the op. */
const RadParamSpec kGemmNtQParams[] = {
    {"M", RAD_P_INT, RAD_REQUIRED, 0},
    {"N", RAD_P_INT, RAD_REQUIRED, 0},
    {"K", RAD_P_INT, RAD_REQUIRED, 0},
    {"group", RAD_P_INT, RAD_REQUIRED, 0},
    {"dtype", RAD_P_STR, RAD_REQUIRED, 0},
    {"pb1", RAD_P_INT, RAD_OPTIONAL, 0},
    {"pb2", RAD_P_INT, RAD_OPTIONAL, 0},
    {"split_n", RAD_P_INT, RAD_OPTIONAL, 0},
};
const RadOperandSpec kGemmNtQOperands[] = {
    {"a", RAD_OPD_IN, 0},
    {"a_scale", RAD_OPD_IN, 1},
    {"b", RAD_OPD_WEIGHT, 0},
    {"b_scale", RAD_OPD_WEIGHT, 0},
    {"y", RAD_OPD_OUT, 0},
    {"a_sum", RAD_OPD_IN, 1},
    {"b_ref", RAD_OPD_WEIGHT, 1},
};

/* quant_act_fp8's schema, as the reference declares it (src/r3d_rows.cpp:615-625). */
const RadParamSpec kQuantActParams[] = {
    {"M", RAD_P_INT, RAD_REQUIRED, 0},
    {"n", RAD_P_INT, RAD_REQUIRED, 0},
    {"group", RAD_P_INT, RAD_REQUIRED, 0},
    {"dtype", RAD_P_STR, RAD_REQUIRED, 0},
};
const RadOperandSpec kQuantActOperands[] = {
    {"x", RAD_OPD_IN, 0},
    {"q", RAD_OPD_OUT, 0},
    {"scale", RAD_OPD_OUT, 0},
};

/* gemm_nt_q_gated's schema (src/r3d_rows.cpp:212-230 of the reference): `act` required, N
 * the weight's rows (twice the gated width), outputs the quantiser's codes and scales. */
const RadParamSpec kGemmGatedParams[] = {
    {"M", RAD_P_INT, RAD_REQUIRED, 0},
    {"N", RAD_P_INT, RAD_REQUIRED, 0},
    {"K", RAD_P_INT, RAD_REQUIRED, 0},
    {"group", RAD_P_INT, RAD_REQUIRED, 0},
    {"dtype", RAD_P_STR, RAD_REQUIRED, 0},
    {"act", RAD_P_STR, RAD_REQUIRED, 0},
};
const RadOperandSpec kGemmGatedOperands[] = {
    {"a", RAD_OPD_IN, 0},
    {"a_scale", RAD_OPD_IN, 0},
    {"b", RAD_OPD_WEIGHT, 0},
    {"b_scale", RAD_OPD_WEIGHT, 0},
    {"q", RAD_OPD_OUT, 0},
    {"scale", RAD_OPD_OUT, 0},
    {"out_bf16", RAD_OPD_OUT, 1},
};

/* gated_quant_fp8's schema (src/r3d_rows.cpp:626-637 of the reference). */
const RadParamSpec kGatedParams[] = {
    {"M", RAD_P_INT, RAD_REQUIRED, 0},
    {"n", RAD_P_INT, RAD_REQUIRED, 0},
    {"group", RAD_P_INT, RAD_REQUIRED, 0},
    {"dtype", RAD_P_STR, RAD_REQUIRED, 0},
    {"act", RAD_P_STR, RAD_OPTIONAL, 0},
};
const RadOperandSpec kGatedOperands[] = {
    {"gate_up", RAD_OPD_IN, 0},
    {"q", RAD_OPD_OUT, 0},
    {"scale", RAD_OPD_OUT, 0},
    {"out_bf16", RAD_OPD_OUT, 1},
};

/* rmsnorm_quant_fp8's schema (src/r3d_rows.cpp:700-716 of the reference). */
const RadParamSpec kRmsParams[] = {
    {"M", RAD_P_INT, RAD_REQUIRED, 0},
    {"n", RAD_P_INT, RAD_REQUIRED, 0},
    {"eps", RAD_P_F64, RAD_REQUIRED, 0},
    {"group", RAD_P_INT, RAD_REQUIRED, 0},
    {"dtype", RAD_P_STR, RAD_REQUIRED, 0},
    {"wadd", RAD_P_F64, RAD_OPTIONAL, 0},
};
const RadOperandSpec kRmsOperands[] = {
    {"x", RAD_OPD_IN, 0},
    {"residual", RAD_OPD_INOUT, 1},
    {"w", RAD_OPD_WEIGHT, 0},
    {"q", RAD_OPD_OUT, 0},
    {"scale", RAD_OPD_OUT, 0},
    {"out_bf16", RAD_OPD_OUT, 1},
};

/* logits_gemm's schema (src/r3d_rows.cpp:233-245 of the reference): gemm_nt's three
 * operands in its order, the extents spelled n_vocab / n_embd. */
const RadParamSpec kLogitsParams[] = {
    {"M", RAD_P_INT, RAD_REQUIRED, 0},
    {"n_vocab", RAD_P_INT, RAD_REQUIRED, 0},
    {"n_embd", RAD_P_INT, RAD_REQUIRED, 0},
    {"dtype", RAD_P_STR, RAD_REQUIRED, 0},
};
const RadOperandSpec kLogitsOperands[] = {
    {"x", RAD_OPD_IN, 0},
    {"lm_head", RAD_OPD_WEIGHT, 0},
    {"logits", RAD_OPD_OUT, 0},
};

const RadOpSchema kSchemas[] = {
    {"gemm_nt_q", kGemmNtQParams, 8, kGemmNtQOperands, 7,
     "Y[M,N] = A[M,K] . dequant(B)[N,K]^T with block-scaled operands; `dtype` names the "
     "operand combination (mxfp4a8: e4m3 A + f32 a_scale per 128 of K, e2m1 B + E8M0 per "
     "32; fp8a8: e4m3 A + f32 a_scale, e4m3 B + bf16 scale per 128 x 128 tile or per row)."},
    {"quant_act_fp8", kQuantActParams, 4, kQuantActOperands, 3,
     "per-(row, `group`-column) symmetric E4M3 quantisation of a token-major activation, "
     "plain row-major; the scale is amax/448, a dequant multiplier (the GEMMs multiply both "
     "scales and never divide)."},
    {"gemm_nt_q_gated", kGemmGatedParams, 6, kGemmGatedOperands, 7,
     "gemm_nt_q over a [2n, K] gate_up weight plane closed by gated_quant_fp8: the outputs are "
     "the quantiser's E4M3 codes, its scale per (row, `group` columns) and optionally the bf16 "
     "gated product; byte-identical to gemm_nt_q followed by gated_quant_fp8."},
    {"gated_quant_fp8", kGatedParams, 5, kGatedOperands, 4,
     "silu(gate)*up or sigmoid(gate)*up (gate the first n columns of each row, up the next "
     "n), narrowed to bf16, then quant_act_fp8's quantiser, in one pass."},
    {"rmsnorm_quant_fp8", kRmsParams, 6, kRmsOperands, 6,
     "RMS norm (optionally after a residual add that is written back) and the fp8 group "
     "quantiser in one pass over the row; the bf16 normed values are what the codes are "
     "taken over, and out_bf16 carries them when present."},
    {"logits_gemm", kLogitsParams, 4, kLogitsOperands, 3,
     "logits[M, n_vocab] = x[M, n_embd] . dequant(lm_head)[n_vocab, n_embd]^T in f32; M "
     "derives from numel(logits) / n_vocab."},
};

/* the band rows' constraint (src/r3d_rows.cpp:1262-1265) */
const RadConstraint cBandMn[] = {
    {"n", RAD_C_GE, 1, nullptr},
    {"dtype", RAD_C_IN, 0, "f32 bf16"},
};

const RadConstraint cMxfp4Tile[] = {
    {"dtype", RAD_C_IN, 0, "mxfp4a8"},
    {"K", RAD_C_DIV, 128, nullptr},
};
const RadConstraint cMxfp4Decode[] = {
    {"dtype", RAD_C_IN, 0, "mxfp4a8"},
    {"M", RAD_C_LE, 16, nullptr},
    {"K", RAD_C_DIV, 128, nullptr},
};
const RadConstraint cMxfp4A16[] = {
    {"dtype", RAD_C_IN, 0, "mxfp4a16"},
    {"K", RAD_C_DIV, 128, nullptr},
};
const RadConstraint cFp8Tile[] = {
    {"dtype", RAD_C_IN, 0, "fp8a8"},
    {"K", RAD_C_DIV, 128, nullptr},
    {"group", RAD_C_EQ, 128, nullptr},
};
const RadConstraint cFp8Decode[] = {
    {"dtype", RAD_C_IN, 0, "fp8a8"},
    {"M", RAD_C_LE, 16, nullptr},
    {"K", RAD_C_DIV, 128, nullptr},
    {"group", RAD_C_EQ, 128, nullptr},
};

/* the gated GEMM row (src/r3d_rows.cpp:1114-1125): the scratch is sized at the band's M
 * bound */
const RadConstraint cFp8Gated[] = {
    {"dtype", RAD_C_IN, 0, "fp8a8"},
    {"M", RAD_C_LE, 64, nullptr},
    {"K", RAD_C_DIV, 128, nullptr},
    {"group", RAD_C_EQ, 128, nullptr},
    {"act", RAD_C_IN, 0, "silu sigmoid"},
};

/* the rmsnorm producer's row (src/r3d_rows.cpp:1419-1423) */
const RadConstraint cRmsQuant[] = {
    {"n", RAD_C_DIV, 4, nullptr},
    {"group", RAD_C_EQ, 128, nullptr},
    {"dtype", RAD_C_IN, 0, "bf16"},
};

/* the e4m3 lm_head row (src/r3d_rows.cpp:1042-1046) */
const RadConstraint cLogitsRow[] = {
    {"n_vocab", RAD_C_GE, 1, nullptr},
    {"n_embd", RAD_C_GE, 128, nullptr},
    {"dtype", RAD_C_IN, 0, "bf16"},
};

enum { kPrioTile = 1000, kPrioDecode = 1100 };

/* The decode rows' levers: split K (waves per weight tile; 0 = the library's policy,
 * which targets ~1280-2048 waves in flight) and the fused producer beyond one row. */
const long long kSplitKValues[] = {0, 1, 2, 4, 8};
const long long kFuseValues[] = {0, 1};
const RadTunable tSplitK[] = {
    {"splitk", kSplitKValues, 5, 0,
     "K chunks per 16-row weight tile, folded through LDS in chunk order; 0 = fill the CUs"},
    {"fuse", kFuseValues, 2, 0,
     "1: bf16 activations (no a_scale) at M = 2..4 are quantised inside the quad GEMV like "
     "the M = 1 call; 0: refused there, so the engine runs quant_act_fp8 first (measured "
     "faster at the 27B decode shapes)"},
};

const RadKernelInfo kRows[] = {
    {"gemm_nt_q_mxfp4", "gemm_nt_q", "gemm",
     "mxfp4a8 prefill GEMM on gfx950 block-scaled MFMA: up to 256 weight rows x 256 tokens "
     "per workgroup, a three-deep direct-to-LDS ring, e2m1 weights with their E8M0 scales "
     "fed to v_mfma_scale_f32_16x16x128_f8f6f4 as is, e4m3 activations, one MFMA per "
     "128-of-K activation group scaled by a_scale in f32; up to M = 128 on a narrow N, K "
     "split across workgroups into f32 partials in launch scratch, summed in chunk order",
     "K a multiple of 128; operands at any alignment (off 16 bytes: the dword-walk arm); "
     "ragged M/N tiles clamp their loads and are never stored; M derives from numel(y)/N; "
     "scratch optional (the hook sizes the split's partials; without them the unsplit arms "
     "run)",
     "fp8_e4m3 a with f32 a_scale per (row, 128 K), e2m1 b with E8M0 b_scale per (row, 32 K), "
     "bf16 y; b_ref accepted and ignored; a_sum refused",
     RAD_DOMAIN_DEVICE, kPrioTile, cMxfp4Tile, 2, nullptr, 0, nullptr,
     nullptr, nullptr, r3d_rad_gemm_nt_q, r3d_rad_gemm_nt_q_scratch, nullptr, nullptr,
     nullptr, nullptr},

    {"gemm_nt_q_mxfp4_decode", "gemm_nt_q", "gemm",
     "mxfp4a8 decode-band GEMV on gfx950: M <= 4 one wave per 4 weight rows (whole 128-byte "
     "lines straight into the MFMA's fp4 operand, E8M0 bytes as its scale operand), M 5..16 "
     "one wave per 32 rows; split-K folded through LDS in chunk order; on planes of 2^26+ "
     "weights past the quad GEMV, K split across workgroups into f32 partials in launch "
     "scratch, summed in chunk order",
     "M <= 16 (decode and speculative verify; widened from the reference's 8); K a multiple "
     "of 128; N any (dead rows clamp their loads and never store); M derives from numel(y)/N; "
     "scratch optional (the hook sizes the split's partials; without them the GEMVs run)",
     "fp8_e4m3 a with f32 a_scale per (row, 128 K), e2m1 b with E8M0 b_scale per (row, 32 K), "
     "bf16 y; b_ref accepted and ignored; a_sum refused",
     RAD_DOMAIN_DEVICE, kPrioDecode, cMxfp4Decode, 3, tSplitK, 2, nullptr,
     nullptr, nullptr, r3d_rad_gemm_nt_q_mxfp4_decode, r3d_rad_gemm_nt_q_mxfp4_decode_scratch,
     nullptr, nullptr, nullptr, nullptr},

    {"gemm_nt_q_fp8a8", "gemm_nt_q", "gemm",
     "fp8a8 prefill GEMM on gfx950 block-scaled MFMA: 128x128 output tile over a three-deep "
     "direct-to-LDS ring, e4m3 on both operands, one MFMA per 128-of-K scale group flushed as "
     "(sub * a_scale) * b_scale in the oracle's order; up to M = 128 on a narrow N, K split "
     "across workgroups into f32 partials in launch scratch, summed in chunk order",
     "K a multiple of 128; operands at any alignment (off 16 bytes: the dword-walk arm); "
     "b_scale either the 128x128 block grid or a per-row grid; M derives from numel(y)/N; "
     "scratch optional (the hook sizes the split's partials; without them the unsplit arms "
     "run)",
     "fp8_e4m3 a with f32 a_scale per (row, 128 K), fp8_e4m3 b with bf16 scale per 128x128 "
     "tile (or per row), bf16 y; a_sum and b_ref refused",
     RAD_DOMAIN_DEVICE, kPrioTile, cFp8Tile, 3, nullptr, 0, nullptr,
     nullptr, nullptr, r3d_rad_gemm_nt_q_fp8, r3d_rad_gemm_nt_q_fp8_scratch, nullptr, nullptr,
     nullptr, nullptr},

    {"gemm_nt_q_fp8a8_decode", "gemm_nt_q", "gemm",
     "fp8a8 decode-band GEMV on gfx950: M <= 4 one wave per 4 weight rows (two whole-line "
     "loads per 128-of-K group into the MFMA's fp8 operand), M 5..16 one wave per 32 rows; "
     "(sub * a_scale) * b_scale per group, split-K folded through LDS in chunk order; on "
     "planes of 2^26+ weights past the quad GEMV, K split across workgroups into f32 partials "
     "in launch scratch, summed in chunk order",
     "M <= 16; K a multiple of 128; N any; b_scale either the 128x128 block grid or a per-row "
     "grid; scratch optional (the hook sizes the split's partials; without them the GEMVs run)",
     "fp8_e4m3 a with f32 a_scale per (row, 128 K), fp8_e4m3 b with bf16 scale per 128x128 "
     "tile (or per row), bf16 y; a_sum and b_ref refused",
     RAD_DOMAIN_DEVICE, kPrioDecode, cFp8Decode, 4, tSplitK, 2, nullptr,
     nullptr, nullptr, r3d_rad_gemm_nt_q_fp8_decode, r3d_rad_gemm_nt_q_fp8_decode_scratch,
     nullptr, nullptr, nullptr, nullptr},

    {"gemm_nt_q_mxfp4a16", "gemm_nt_q", "gemm",
     "mxfp4 prefill GEMM with bf16 activations on gfx950: the activations are quantised to "
     "mxfp8 (e4m3 + E8M0 per 32 of K) into launch scratch, then both E8M0 planes ride in "
     "v_mfma_scale_f32_16x16x128_f8f6f4, which accumulates in place; up to 256 x 256 "
     "output tile per workgroup over a three-deep direct-to-LDS ring",
     "K a multiple of 128; a_scale absent; launch scratch >= M*K (rounded to 256) + M*K/32 "
     "bytes, 16-byte aligned (the row's scratch hook sizes it from M and K); A and B at any "
     "alignment (off 16 bytes: the element-wise quantiser / dword-walk arm); M derives from "
     "numel(y)/N",
     "bf16 a, e2m1 b with E8M0 b_scale per (row, 32 K), bf16 y; b_ref accepted and ignored; "
     "a_scale and a_sum refused",
     RAD_DOMAIN_DEVICE, kPrioTile, cMxfp4A16, 2, nullptr, 0, nullptr,
     nullptr, nullptr, r3d_rad_gemm_nt_q_mxfp4a16, r3d_rad_gemm_nt_q_mxfp4a16_scratch,
     nullptr, nullptr, nullptr, nullptr},

    {"quant_act_fp8_act", "quant_act_fp8", "band",
     "per-group symmetric E4M3 quantisation of an activation, plain row-major, on gfx950: one "
     "wave per (row, group), v_max_f32 maximum over the group, v_cvt_pk_fp8_f32 encode",
     "f32/bf16 inputs; the scale is amax/448, a dequant multiplier; group clamped to n; at "
     "most 65535 rows",
     "activation in, f8e4m3 codes and f32 group scales out",
     RAD_DOMAIN_DEVICE, kPrioTile, cBandMn, 2, nullptr, 0, nullptr,
     nullptr, nullptr, r3d_rad_quant_act_fp8, nullptr, nullptr, nullptr, nullptr, nullptr},

    {"gated_quant_fp8_act", "gated_quant_fp8", "band",
     "silu(gate)*up or sigmoid(gate)*up fused with quant_act_fp8's quantiser on gfx950: one "
     "workgroup per row with 8 elements a lane for groups of 8..512 that tile the row, else "
     "one wave per (row, group) recomputing the gated value for its encode pass",
     "f32/bf16 gate_up [M, 2n]; the gated value narrows to bf16 once (exp in double, as the "
     "reference's sigmoid); group clamped to n; at most 65535 rows",
     "f32/bf16 gate_up in, f8e4m3 codes, f32 scales, optional bf16/f32 gated output",
     RAD_DOMAIN_DEVICE, kPrioTile, cBandMn, 2, nullptr, 0, nullptr,
     nullptr, nullptr, r3d_rad_gated_quant_fp8, nullptr, nullptr, nullptr, nullptr, nullptr},

    {"rmsnorm_quant_fp8", "rmsnorm_quant_fp8", "quant",
     "RMS norm and the fp8 group quantiser on gfx950: one workgroup of 256 lanes per row, the "
     "row staged in LDS as bf16, the sum of squares folded in the reference's order (lane "
     "strides of 256, 32-lane shuffle trees, eight partials in order), one wave per group",
     "n <= 30720 (the row in LDS); w rank 1; with a residual the bf16-narrowed sum is stored "
     "before the variance reads it; at most 65535 rows",
     "bf16 in (and residual), f32/bf16 w, fp8_e4m3 codes with an f32 per-group scale, "
     "optional bf16/f32 out_bf16",
     RAD_DOMAIN_DEVICE, kPrioTile, cRmsQuant, 3, nullptr, 0, nullptr,
     nullptr, nullptr, r3d_rad_rmsnorm_quant_fp8, nullptr, nullptr, nullptr, nullptr, nullptr},

    {"gemm_nt_q_gated_fp8a8", "gemm_nt_q_gated", "gemm",
     "the fp8a8 GEMM (decode GEMV up to M = 16, the prefill pipeline above) writing its bf16 "
     "gate_up plane into the launch scratch, closed by the gated_quant_fp8 kernels on the same "
     "stream -- the byte-identical composition of the two rows",
     "M <= 64 (the scratch is sized at the band's bound, 64*N*2 bytes, 16-byte aligned); K a "
     "multiple of 128; N = 2n; M derives from numel(q)/n",
     "fp8_e4m3 a with f32 a_scale per (row, 128 K), fp8_e4m3 b with bf16 scale per 128x128 "
     "tile (or per row), e4m3 q + f32 scale out, optional bf16/f32 gated product; act silu "
     "or sigmoid; a_sum refused",
     RAD_DOMAIN_DEVICE, kPrioTile, cFp8Gated, 5, nullptr, 0, nullptr,
     nullptr, nullptr, r3d_rad_gemm_nt_q_gated_fp8, r3d_rad_gemm_nt_q_gated_fp8_scratch,
     nullptr, nullptr, nullptr, nullptr},

    /* The layout hooks (r3d_head.cpp) admit exactly the joined e4m3 + block-scale head the
     * launch reads and answer with the canonical rad.planes join; a plain head is declined
     * at declare time (this library has no bf16 head row to claim it first). */
    {"logits_gemm_e4m3", "logits_gemm", "vocab",
     "lm_head GEMV on gfx950 bf16 MFMA: e4m3 codes widened exactly to bf16 in registers "
     "(v_cvt_scalef32_pk_bf16_fp8), 16 activation rows staged once per workgroup in LDS, "
     "16 head rows per MFMA streamed from HBM with 16-byte buffer loads, the block scale "
     "applied once per 128-column window in f32",
     "codes [n_vocab, n_embd] e4m3 dense, scale per (1 or 128 rows, 128 cols); n_embd a "
     "multiple of 4 up to 40448 (off a multiple of 16, or x / codes / scale off alignment: "
     "a slower dword walk); M derives from numel(logits)/n_vocab, up to 8 rows a pass (fewer "
     "where LDS holds fewer rows of n_embd), passes ride grid.y",
     "bf16 x, joined e4m3 + bf16/f16/f32 head (rad.planes), f32 logits",
     RAD_DOMAIN_DEVICE, kPrioTile, cLogitsRow, 3, nullptr, 0, nullptr,
     nullptr, nullptr, r3d_rad_logits_gemm_e4m3, nullptr, r3d_layout_head, r3d_relayout_head,
     nullptr, r3d_unrelayout_head},
};

bool row_hidden(const RadKernelInfo& k) {
    const bool no_mx = r3d::env_no_mxfp4(), no_mxd = r3d::env_no_fp4_dec();
    const bool no_f8 = r3d::env_no_fp8a8(), no_f8d = r3d::env_no_fp8_dec();
    if (!strcmp(k.name, "gemm_nt_q_mxfp4")) return no_mx;
    if (!strcmp(k.name, "gemm_nt_q_mxfp4a16")) return no_mx;
    if (!strcmp(k.name, "gemm_nt_q_mxfp4_decode")) return no_mx || no_mxd;
    if (!strcmp(k.name, "gemm_nt_q_fp8a8")) return no_f8;
    if (!strcmp(k.name, "gemm_nt_q_gated_fp8a8")) return no_f8;
    if (!strcmp(k.name, "gemm_nt_q_fp8a8_decode")) return no_f8 || no_f8d;
    return false;
}

}  // namespace

extern "C" {

uint32_t rad_plugin_abi_version(void) { return RAD_ABI_VERSION; }

const RadPluginInfo* rad_plugin_info(void) {
    static const RadPluginInfo info = {
        RAD_PLUGIN_KERNEL, "libr3d_gfx950", "0.1.0",
        "radiance gemm_nt_q rows (mxfp4a8, fp8a8, mxfp4a16), gemm_nt_q_gated (fp8a8), the "
        "e4m3 logits_gemm lm_head and the quant_act_fp8 / gated_quant_fp8 / "
        "rmsnorm_quant_fp8 producers for "
        "AMD Instinct MI355X (CDNA4)",
        "gfx950",
    };
    return &info;
}

int rad_kernel_schema_count(void) { return (int)(sizeof kSchemas / sizeof kSchemas[0]); }

const RadOpSchema* rad_kernel_schema_at(int i) {
    if (i < 0 || i >= rad_kernel_schema_count()) return nullptr;
    return &kSchemas[i];
}

int rad_kernel_count(void) {
    int n = 0;
    for (const RadKernelInfo& k : kRows)
        if (!row_hidden(k)) ++n;
    return n;
}

const RadKernelInfo* rad_kernel_at(int i) {
    if (i < 0) return nullptr;
    for (const RadKernelInfo& k : kRows)
        if (!row_hidden(k) && i-- == 0) return &k;
    return nullptr;
}

/* The build script passes the sources' SHA-256 as R3D_BUILD_ID; a compile without it
 * reports "unknown". */
#ifndef R3D_BUILD_ID
#define R3D_BUILD_ID "unknown"
#endif
const char* r3d_gfx950_build_id(void) { return R3D_BUILD_ID; }

}  /* extern "C" */
