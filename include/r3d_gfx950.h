/* r3d_gfx950.h -- the C ABI exported by libr3d_gfx950.so.
 *
 * Every entry point replaces the reference libr3d export of the same name; the engine
 * (radiance, ABI 26) dlopens the library, reads the row table through the rad_* calls
 * and reaches the gemm_nt_q entries through RadKernelInfo::launch.  Plain C types and
 * device pointers only.
 */
#ifndef R3D_GFX950_H
#define R3D_GFX950_H

#include <stdint.h>
#include "rad_abi.h"
#include "rad_planes.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Plugin identity.  Replaces src/r3d_rows.cpp:16 (returns RAD_ABI_VERSION, 26) and
 * src/r3d_rows.cpp:18-27 (name, version, description, targets "gfx950"). */
uint32_t rad_plugin_abi_version(void);
const RadPluginInfo* rad_plugin_info(void);

/* Op schemas this plugin declares: gemm_nt_q (src/r3d_rows.cpp:186-210) and quant_act_fp8
 * (src/r3d_rows.cpp:615-625,985-990), parameters and operands exactly as there.
 * Replaces src/r3d_rows.cpp:2238-2247. */
int rad_kernel_schema_count(void);
const RadOpSchema* rad_kernel_schema_at(int i);

/* The row table after the registration-time kill switches (R3D_NO_MXFP4,
 * R3D_NO_FP4_DEC, R3D_NO_FP8A8, R3D_NO_FP8_DEC).  Replaces src/r3d_rows.cpp:2266-2278
 * with the gate of src/r3d_rows.cpp:2216-2236. */
int rad_kernel_count(void);
const RadKernelInfo* rad_kernel_at(int i);

/* gemm_nt_q at mxfp4a8, prefill row (any M).  Replaces src/r3d_gemm_mxfp4.hip:1587-1691.
 * Operands (a, a_scale, b, b_scale, y, a_sum?, b_ref?); params N, K, dtype "mxfp4a8";
 * M = numel(y)/N.  Returns RAD_OK, or RAD_E_UNSUPPORTED / RAD_E_SHAPE / RAD_E_STRIDE for a
 * refused format and RAD_E_DEVICE for a failed launch.  Asynchronous on `s`. */
int r3d_rad_gemm_nt_q(const RadArgs* a, RadStream s);

/* gemm_nt_q at mxfp4a8, decode band M <= 16.  Replaces src/r3d_gemm_mxfp4.hip:1712-2170
 * (r3d_rad_gemm_nt_q_mxfp4_decode and its q8x sibling share this one row here).  Beyond the
 * reference: at M = 1 it also takes a bf16 activation row with a_scale absent and quantises
 * it as quant_act_fp8 does (src/r3d_band.hip:117-153) before the products. */
int r3d_rad_gemm_nt_q_mxfp4_decode(const RadArgs* a, RadStream s);

/* gemm_nt_q at fp8a8, prefill row.  Replaces src/r3d_gemm_fp8a8.hip:1054-1099. */
int r3d_rad_gemm_nt_q_fp8(const RadArgs* a, RadStream s);

/* Scratch hooks (RadKernelInfo::scratch) of the two tile rows, r3d_rad_gemm_nt_q (mxfp4a8)
 * and r3d_rad_gemm_nt_q_fp8.  No counterpart in the reference, whose tile rows take no
 * scratch: up to M = 128 on an N too narrow to fill the chip with 128-row tiles, these rows
 * split K across workgroups into f32 partial planes in RadArgs::scratch and sum them in
 * order on the same stream.  The hook returns the bytes of those planes (kc * M * N * 4 at
 * the N and K parameters and M = numel(y) / N -- without y the M parameter, else 128), 0 when no split applies.
 * The scratch is optional: a launch without it, or with less, or at an address that is not
 * 16-byte aligned, runs the unsplit arms (never a refusal). */
int64_t r3d_rad_gemm_nt_q_scratch(const RadArgs* a);
int64_t r3d_rad_gemm_nt_q_fp8_scratch(const RadArgs* a);

/* gemm_nt_q at fp8a8, decode band M <= 16.  Replaces src/r3d_gemm_fp8a8.hip:1101-1130.
 * Takes a bf16 activation row at M = 1 as the mxfp4a8 decode entry does. */
int r3d_rad_gemm_nt_q_fp8_decode(const RadArgs* a, RadStream s);

/* Scratch hooks (RadKernelInfo::scratch) of the two decode rows, r3d_rad_gemm_nt_q_mxfp4_decode
 * and r3d_rad_gemm_nt_q_fp8_decode.  No counterpart in the reference, whose decode rows take
 * no scratch: where the quad GEMV does not take the launch (M = 5..16, or an M <= 4 shape
 * whose activation rows it cannot stage) on a plane of at least 2^26 weights, and no
 * "splitk" tunable pins the GEMV's split, these rows split K across workgroups into f32
 * partial planes in RadArgs::scratch and sum them in order on the same stream.  The hook
 * returns the bytes of those planes (kc * M * N * 4 at the N and K parameters and M =
 * numel(y) / N -- without y the M parameter, else 16), 0 when no split applies.  The
 * scratch is optional: a launch without it, or with less, or at an address that is not
 * 16-byte aligned, runs the decode GEMVs (never a refusal). */
int64_t r3d_rad_gemm_nt_q_mxfp4_decode_scratch(const RadArgs* a);
int64_t r3d_rad_gemm_nt_q_fp8_decode_scratch(const RadArgs* a);

/* gemm_nt_q at dtype "mxfp4a16", prefill row (any M).  No counterpart in the reference:
 * the bf16-activation variant of the mxfp4 prefill (a bf16 [M, K], a_scale absent,
 * weights as mxfp4a8), for engines that feed unquantised activations.  The launch
 * quantises a to mxfp8 (e4m3 + E8M0 per 32 of K) into RadArgs::scratch, then runs the
 * block-scaled MFMA GEMM; both kernels run on `s`.  The launch-signature convention is
 * src/r3d_gemm_mxfp4.hip:1587-1588; the scratch refusal follows
 * src/r3d_gemm_fp8a8.hip:1214-1218 (RAD_E_UNSUPPORTED when scratch is missing or short). */
int r3d_rad_gemm_nt_q_mxfp4a16(const RadArgs* a, RadStream s);

/* The mxfp4a16 row's scratch hook (RadKernelInfo::scratch): bytes of launch scratch for
 * the M and K parameters, 0 when either is missing.  Same role as the reference's
 * src/r3d_gemm_fp8a8.hip:1249-1253. */
int64_t r3d_rad_gemm_nt_q_mxfp4a16_scratch(const RadArgs* a);

/* quant_act_fp8, the activation producer of the fp8a8 / mxfp4a8 rows: per-(row, group)
 * symmetric e4m3 codes of a bf16 or f32 activation, plain row-major, and the f32 dequant
 * scale amax/448 per group.  Operands (x, q, scale); params M, n, group, dtype.  Replaces
 * src/r3d_band.hip:460-487 (gates and refusal codes as there: RAD_E_INVAL for a missing
 * operand, RAD_E_DTYPE, RAD_E_SHAPE, RAD_E_STRIDE; RAD_E_DEVICE for a failed launch).
 * Asynchronous on `s`. */
int r3d_rad_quant_act_fp8(const RadArgs* a, RadStream s);

/* gated_quant_fp8: silu(gate) * up (or sigmoid(gate) * up), narrowed to bf16, then the
 * quant_act_fp8 quantiser.  Replaces src/r3d_band.hip:489-547 (r3d_rad_gated_quant_fp8). */
int r3d_rad_gated_quant_fp8(const RadArgs* a, RadStream s);

/* rmsnorm_quant_fp8: RMS norm (after an optional residual add written back) and the fp8
 * group quantiser over the bf16 normed row.  Replaces src/r3d_more.hip:479-539
 * (r3d_rad_rmsnorm_quant_fp8). */
int r3d_rad_rmsnorm_quant_fp8(const RadArgs* a, RadStream s);

/* gemm_nt_q_gated at fp8a8: the fp8a8 GEMM into the launch scratch, then gated_quant_fp8
 * over it.  Replaces src/r3d_gemm_fp8a8.hip:1163-1241 (r3d_rad_gemm_nt_q_gated_fp8). */
int r3d_rad_gemm_nt_q_gated_fp8(const RadArgs* a, RadStream s);

/* The gated row's scratch hook: 64 * N * 2 bytes (0 without N).  Replaces
 * src/r3d_gemm_fp8a8.hip:1246-1253 (r3d_rad_gemm_nt_q_gated_fp8_scratch). */
int64_t r3d_rad_gemm_nt_q_gated_fp8_scratch(const RadArgs* a);

/* logits_gemm over a joined e4m3 + block-scale head: bf16 x [M, n_embd], lm_head a
 * joined-planes blob (rad_planes.h: "codes" e4m3 [n_vocab, n_embd] dense, "scale" bf16 /
 * f16 / f32 per (1 or 128 rows, 128 columns)), f32 logits [M, n_vocab], M =
 * numel(logits) / n_vocab.  Replaces src/r3d_gemm_logits.hip:144-226
 * (r3d_rad_logits_gemm_e4m3).  n_embd a multiple of 4 at any alignment of x, codes and
 * scale (off a multiple of 16 or off 16-byte alignment: a slower dword walk).  The first
 * launch over a blob in device memory reads its header and entries with a copy on the
 * launch stream and waits for it (cached per device and address; refused with
 * RAD_E_UNSUPPORTED under graph capture -- launch once first); see
 * r3d_gfx950_logits_head_forget. */
int r3d_rad_logits_gemm_e4m3(const RadArgs* a, RadStream s);

/* The logits_gemm_e4m3 row's weight-layout hooks (host only).  Replace
 * src/r3d_gemm_logits.hip:233-272 (r3d_layout_head / r3d_relayout_head /
 * r3d_unrelayout_head, registered at src/r3d_rows.cpp:1598-1599).  They admit the head
 * (operand 1) as an untransformed "affine" encoding whose selected planes are "codes"
 * (tiled 1 x 1, e4m3, [n_vocab, n_embd]) then "scale" (tiled bf16 / f16 / f32, block
 * (1 or 128) x 128, [ceil(n_vocab / block), ceil(n_embd / 128)]) with n_embd a multiple of
 * 4 the launch can stage, and answer with the canonical rad.planes join (rad_planes.h):
 * layout gives its tag and bytes, relayout writes it into host memory dst, unrelayout
 * reads the planes back.  Any other operand: RAD_E_UNSUPPORTED (stored as is); any other
 * head, a plain one without that encoding included: declined (RAD_E_DTYPE, or RAD_E_SHAPE
 * for grids that disagree). */
int r3d_layout_head(const RadParam* p, int n_p, int operand, const RadEncoding* enc,
                    const int* sel, const RadTensor* planes, int n, RadLayout* out);
int r3d_relayout_head(const RadParam* p, int n_p, int operand, const RadEncoding* enc,
                      const int* sel, const RadTensor* planes, int n, void* dst,
                      int64_t dst_bytes);
int r3d_unrelayout_head(const RadParam* p, int n_p, int operand, const RadEncoding* enc,
                        const int* sel, const void* src, int64_t src_bytes,
                        const RadTensor* planes, int n);

/* The same join for a caller holding the two planes directly, no counterpart in the
 * reference (it is what r3d_relayout_head writes for the head's encoding), in host memory:
 *   _bytes: the blob's size for n_vocab x n_embd codes and a scale plane of scale_dtype
 *           (RAD_BF16 / RAD_F16 / RAD_F32) with scale_block_rows (1 or 128) rows per
 *           element, or a negative RAD_E_* code;
 *   _header: the same, and the blob's header and entries into *out (the planes go at the
 *           entries' offsets: a caller can stream them straight into device memory);
 *   _join:  writes header, entries, codes (rows codes_pitch bytes apart) and scale (rows
 *           scale_pitch_bytes apart, (n_embd + 127) / 128 elements each) into dst;
 *   _split: the inverse, into dense planes (either pointer may be null), after checking
 *           each plane's dtype, grid, pitch and extent against the blob; the planes take
 *           the blob's own grids (codes rows x cols bytes, scale rows x cols elements, as
 *           its entries state: read them first, _header or rad_planes_find, to size the
 *           destinations). */
int64_t r3d_gfx950_logits_head_bytes(int64_t n_vocab, int64_t n_embd, uint32_t scale_dtype,
                                     int64_t scale_block_rows);
int64_t r3d_gfx950_logits_head_header(int64_t n_vocab, int64_t n_embd, uint32_t scale_dtype,
                                      int64_t scale_block_rows, RadPlanesHead* out);
int r3d_gfx950_logits_head_join(const uint8_t* codes, int64_t codes_pitch, const void* scale,
                                int64_t scale_pitch_bytes, int64_t n_vocab, int64_t n_embd,
                                uint32_t scale_dtype, int64_t scale_block_rows, void* dst,
                                int64_t dst_bytes);
int r3d_gfx950_logits_head_split(const void* blob, int64_t blob_bytes, uint8_t* codes,
                                 void* scale);

/* No counterpart in the reference: drops the cached header of the blob at `blob` (every
 * device).  Call it before a different head is joined at an address a launch has used;
 * a launch whose cached header no longer matches the device's writes NaN logits. */
void r3d_gfx950_logits_head_forget(const void* blob);

/* gemm_nt_q at dtype "mxfp4a16" that allocates nothing: no counterpart in the reference,
 * for callers that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same operands, parameters, kernels and results as
 * r3d_rad_gemm_nt_q_mxfp4a16, but RadArgs::scratch is not used: the quantised activations
 * go to a static device buffer of R3D_NOALLOC_SCRATCH_BYTES per GPU, held until the
 * process ends.  A call needing more (round256(M*K) + M*K/32 bytes) is refused with
 * RAD_E_SHAPE and a line on stderr.  All calls on one GPU share its buffer: calls that
 * overlap on one GPU (other streams, other threads) race. */
#define R3D_NOALLOC_SCRATCH_BYTES (16ll << 20)
int r3d_rad_gemm_nt_q_mxfp4a16_noalloc(const RadArgs* a, RadStream s);

/* Host-only diagnostic with no counterpart in the reference: runs `row`'s preamble and
 * plan on `a` and writes the chosen arm and launch geometry (or the refusal) into buf.
 * Launches nothing and copies nothing from the device: a logits head's header is read in
 * place when the blob is host-accessible, else taken from the copy an earlier launch
 * cached (RAD_E_UNSUPPORTED when there is none).  Returns the plan's status code. */
int r3d_gfx950_describe(const char* row, const RadArgs* a, char* buf, int len);

/* Diagnostic with no counterpart in the reference: one stage of a gemm_nt_q_mxfp4a16 call
 * on `s`, for timing and checking the stages apart.  stage 0 = the whole call (as the
 * row's launch), 1 = the mxfp8 quantiser alone (fills RadArgs::scratch), 2 = the
 * block-scaled GEMM alone on the planes already in RadArgs::scratch.  Same gates and
 * refusal codes as the row; RAD_E_INVAL for another stage; RAD_E_UNSUPPORTED where the
 * call would take the skinny band's decode passes (no quantiser stage there). */
int r3d_gfx950_mxfp4a16_stage(const RadArgs* a, RadStream s, int stage);

/* Measurement diagnostic with no counterpart in the reference: a read-only stream over
 * `bytes` of device memory at src on `s` -- each wave one contiguous run of kb KB read by
 * 1 KB loads (64 lanes x 16 bytes, non-temporal) kept 8 deep in flight, waves_per_wg
 * (1..8) waves a workgroup -- the ceiling an HBM-bound kernel of that access pattern and
 * size is held against.  bytes = 0 launches kb waves that do nothing (the launch floor).
 * sink: a device dword written only if the XOR of the data hits a fixed value.  RAD_OK,
 * RAD_E_INVAL for a bad argument, RAD_E_DEVICE if the launch fails. */
int r3d_gfx950_stream_probe(const void* src, int64_t bytes, int waves_per_wg, int64_t kb,
                            uint32_t* sink, RadStream s);

/* Measurement diagnostic with no counterpart in the reference: one wave on `s` runs `iters`
 * rounds of four 16 x 16 x 128 e4m3 MFMAs (four in-place accumulator chains) with `nv`
 * independent f32 fused multiply-adds before each (nv 0, 4, 8 or 16; with lag3 != 0, 4 or 8
 * multiply-adds that read the result of the MFMA issued three earlier), and writes the
 * shader-clock ticks the loop took to the device int64 at `cycles`.  work: a device buffer
 * of at least 1 KB (inputs read from its first 512 bytes, results written after them).
 * Divided by 4 * iters it gives the cost of one MFMA plus its share of VALU work: how much
 * VALU a wave hides under its own MFMAs.  RAD_OK, RAD_E_INVAL for a bad argument,
 * RAD_E_DEVICE if the launch fails. */
int r3d_gfx950_mfma_valu_probe(int nv, int lag3, int iters, void* work, int64_t* cycles,
                               RadStream s);

/* Build identity with no counterpart in the reference: the SHA-256 (hex) of the compile
 * flags and of the sources this library was compiled from -- the flags as one line, then
 * every file under libr3d_amd/csrc and include, in name order, each as "<relative
 * path>\n<bytes>" -- so a test harness can tell whether the binary it loaded was built
 * from the tree beside it. */
const char* r3d_gfx950_build_id(void);

#ifdef __cplusplus
}
#endif

#endif /* R3D_GFX950_H */
