/* r3d_oracle.h -- CPU restatement of radiance libref's gemm_nt_q arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker or the timed CPU
 * baseline -- never as the product path.  The product (libr3d_amd/libr3d_gfx950.so)
 * does not link or call anything here.
 *
 * The real oracle, libref (radiance v1.11.0: ref_gemm.h quant_dot / grid_block /
 * row_stride, ref_quant.cpp, rad_plugin.h's rad_fp8e4m3_to_f32 / rad_fp4e2m1_to_f32 /
 * rad_f32_to_fp8e4m3), lives outside the reference tree and cannot be built here
 * (reference Dockerfile clones it from the network: docker/Dockerfile.dev:16,25-26).
 * Every function below restates the reference's own transcription of it, cited per
 * function.  Compiled with -ffp-contract=off, as the reference compiles its
 * arithmetic (CMakeLists.txt:34-63).
 *
 * Pinning (what each function is checked against) is listed in the header comment of
 * r3d_oracle.c.
 */
#ifndef R3D_ORACLE_H
#define R3D_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* scalar codecs */
float    r3d_ref_e4m3_to_f32(uint8_t b);
float    r3d_ref_e2m1_to_f32(uint8_t nibble);
float    r3d_ref_e8m0_to_f32(uint8_t x);
uint8_t  r3d_ref_f32_to_e4m3(float f);
uint16_t r3d_ref_f32_to_bf16(float f);
float    r3d_ref_bf16_to_f32(uint16_t h);

/* bulk codecs (for exhaustive / vector checks from Python) */
void r3d_ref_e4m3_to_f32_n(const uint8_t* in, float* out, int64_t n);
void r3d_ref_f32_to_e4m3_n(const float* in, uint8_t* out, int64_t n);
void r3d_ref_f32_to_bf16_n(const float* in, uint16_t* out, int64_t n);
/* dequantised mxfp4 weights: out[n*K + k] = e2m1(code) * e8m0(scale), f32 */
void r3d_ref_mxfp4_dequant(const uint8_t* B, const uint8_t* BS, int64_t N, int64_t K,
                           int64_t bs_pitch, float* out);

/* libref grid_block / row_stride helpers (host shape rules) */
int64_t r3d_ref_grid_block(int64_t ext, int64_t blocks);

/* quant_act_fp8: x [M, K] (bf16 when x_is_bf16, else f32) with row pitch x_pitch
 * (elements) -> q [M, K] e4m3 (pitch q_pitch) and scale [M, ceil(K/group)] f32
 * (pitch s_pitch). */
void r3d_ref_quant_act_fp8(const void* x, int x_is_bf16, int64_t M, int64_t K,
                           int64_t x_pitch, int64_t group, uint8_t* q, int64_t q_pitch,
                           float* scale, int64_t s_pitch);

/* gated_quant_fp8: gate_up [M, 2n] (bf16 when gu_is_bf16, else f32), row pitch gu_pitch;
 * silu selects x*sigmoid(x) over sigmoid(x); codes q [M, n], scales [M, ceil(n/group)];
 * out (nullable) the gated value's bf16 bits [M, n]. */
void r3d_ref_gated_quant_fp8(const void* gu, int gu_is_bf16, int64_t M, int64_t n,
                             int64_t gu_pitch, int64_t group, int silu, uint8_t* q,
                             int64_t q_pitch, float* scale, int64_t s_pitch, uint16_t* out,
                             int64_t out_pitch);

/* rmsnorm_quant_fp8: x bf16 [M, n] (row pitch x_pitch); res (nullable) bf16 [M, n] updated
 * with bf16(res + x); w [n] (bf16 when w_is_bf16, else f32); codes q [M, n], scales
 * [M, ceil(n/group)]; out (nullable) the normed values' bf16 bits [M, n]. */
void r3d_ref_rmsnorm_quant_fp8(const uint16_t* x, int64_t M, int64_t n, int64_t x_pitch,
                               uint16_t* res, int64_t r_pitch, const void* w, int w_is_bf16,
                               int64_t group, float eps, float wadd, uint8_t* q,
                               int64_t q_pitch, float* scale, int64_t s_pitch, uint16_t* out,
                               int64_t out_pitch);

/* quant_dot at mxfp4a8.
 *   A  [M, K] e4m3 (pitch a_pitch bytes), AS [M, ceil(K/128)] f32 (pitch as_pitch)
 *   B  [N, K/2] packed e2m1, low nibble = even k (pitch K/2 bytes)
 *   BS [N, ceil(K/32)] E8M0 (pitch bs_pitch)
 *   Y  [M, N] bf16 (pitch y_pitch); Yf (optional) the f32 accumulator; S (optional) the
 *   per-element magnitude sum  sum_g |sum_k |a*b|| * |sa| * |sb|  used for error bounds.
 * nthreads <= 1 runs serially; otherwise OpenMP over output rows n. */
void r3d_ref_quant_dot_mxfp4a8(const uint8_t* A, int64_t a_pitch, const float* AS,
                               int64_t as_pitch, const uint8_t* B, const uint8_t* BS,
                               int64_t bs_pitch, int64_t M, int64_t N, int64_t K,
                               uint16_t* Y, int64_t y_pitch, float* Yf, float* S,
                               int nthreads);

/* quant_dot at fp8a8.  B [N, K] e4m3 (pitch b_pitch); BS bf16 with rblk 1 ([N, K/128],
 * per-row grid) or rblk 128 ([ceil(N/128), K/128], the 128x128 block grid). */
void r3d_ref_quant_dot_fp8a8(const uint8_t* A, int64_t a_pitch, const float* AS,
                             int64_t as_pitch, const uint8_t* B, int64_t b_pitch,
                             const uint16_t* BS, int64_t bs_pitch, int rblk,
                             int64_t M, int64_t N, int64_t K,
                             uint16_t* Y, int64_t y_pitch, float* Yf, float* S,
                             int nthreads);

/* The mxfp8 activation quantiser of the bf16-activation prefill row (no counterpart in
 * the reference; OCP MX v1.0 block format, E8M0 scale per 32 of K): per (row, 32 of K)
 * block the scale exponent e is the least integer with amax * 2^-e <= 448 (so no code
 * saturates; an all-zero block takes e = 0), clamped to [-127, 127], scale byte e + 127,
 * and codes q = f32_to_e4m3(x * 2^-e), RTNE.  x is bf16. */
void r3d_ref_quant_act_mxfp8(const uint16_t* x, int64_t M, int64_t K, int64_t x_pitch,
                             uint8_t* q, int64_t q_pitch, uint8_t* sx, int64_t sx_pitch);

/* Dot of mxfp8 activations with mxfp4 weights, both block-scaled per 32 of K:
 *   acc = sum_g (sum_{k in g} a_k*b_k) * 2^(xa_g-127) * 2^(xb_g-127) -> bf16.
 * S as above. */
void r3d_ref_dot_mx8_mxfp4(const uint8_t* A, int64_t a_pitch, const uint8_t* SX,
                           int64_t sx_pitch, const uint8_t* B, const uint8_t* BS,
                           int64_t bs_pitch, int64_t M, int64_t N, int64_t K,
                           uint16_t* Y, int64_t y_pitch, float* Yf, float* S,
                           int nthreads);

/* Error model of the gfx950 block-scaled MFMA (a test-side quantity, not part of libref):
 * the matrix core sums the products of every 8 consecutive k at a width aligned to the
 * group's largest product and truncates bits below 2^-13 of it (measured on MI355X), so
 * a kernel built on it can differ from the exact product by up to 7 * 2^-13 of each
 * group's largest |a*b| * |sa| * |sb|.  S8[m, n] = sum over 8-groups of that maximum.
 * enc 0 = mxfp4a8 operands (BS E8M0), 1 = fp8a8 operands (BS bf16, rblk), 2 = mxfp4
 * weights with activation scales per 32 of K (AS holds the decoded E8M0 values). */
void r3d_ref_group8_mag(int enc, const uint8_t* A, int64_t a_pitch, const float* AS,
                        int64_t as_pitch, const uint8_t* B, int64_t b_pitch, const void* BS,
                        int64_t bs_pitch, int rblk, int64_t M, int64_t N, int64_t K,
                        float* S8, int nthreads);

/* Wall-clock helper for the CPU baseline: number of OpenMP threads available. */
int r3d_ref_max_threads(void);

/* IEEE binary16 bits -> f32, exact (subnormals, infinities and NaN kept). */
float r3d_ref_f16_to_f32(uint16_t h);

/* logits_gemm over a joined e4m3 head.
 *   x      [M, K] bf16 bits, row pitch x_pitch (elements)
 *   codes  [N, K] e4m3, dense
 *   scale  [ceil(N/br), ceil(K/128)] of sdt (0 bf16 bits, 1 f16 bits, 2 f32), row pitch
 *          s_pitch (elements); br 1 or 128
 *   Y      [M, N] f32 (pitch y_pitch); S (optional) [M, N] the magnitude sum
 *          sum_k |x * (code * s)| accumulated in f32, for error bounds. */
void r3d_ref_logits_e4m3(const uint16_t* x, int64_t x_pitch, const uint8_t* codes,
                         const void* scale, int sdt, int64_t s_pitch, int br, int64_t M,
                         int64_t N, int64_t K, float* Y, int64_t y_pitch, float* S,
                         int nthreads);

#ifdef __cplusplus
}
#endif

#endif /* R3D_ORACLE_H */
