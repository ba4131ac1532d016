/* r3d_oracle.c -- CPU restatement of libref's gemm_nt_q (mxfp4a8, fp8a8) and of the
 * quant_act_fp8 producer.  TEST INFRASTRUCTURE: see r3d_oracle.h for who may use it.
 *
 * Built with  -O3 -ffp-contract=off -fopenmp  (oracle/Makefile).  No -ffast-math: the
 * quantiser's 1/scale and x*inv must be correctly rounded IEEE f32 operations.
 *
 * What pins each function (tests/test_oracle.py):
 *   e4m3 decode     exhaustive 256 codes vs torch.float8_e4m3fn (a library, not the
 *                   reference); NaN compared as a class.
 *   e2m1 decode     all 16 codes vs the closed form sign*(e==0 ? m/2 : (1+m/2)*2^(e-1)).
 *   e8m0 decode     all 256 bytes vs torch.float8_e8m0fnu and ldexp(1, x-127).
 *   e4m3 encode     vs torch inside +-448 (torch does not saturate) on every f32 whose
 *                   exponent lies in the e4m3 range plus random patterns; vs a
 *                   nearest-value search over the decoded code table (round half to
 *                   even code) on all ties and midpoints; saturation and NaN by value.
 *   bf16 RNE        vs torch's float32 -> bfloat16 conversion on random and special
 *                   patterns (NaN as a class: this restatement keeps sign and payload).
 *   grid_block      closed forms: exact grids (K/b columns) return b; 1 column -> ext.
 *   quant_act_fp8   invariants: the amax element encodes to +-448, zero groups take
 *                   scale 1 and code 0, |dequant - x| <= half an e4m3 ulp relative,
 *                   NaN inputs encode to the NaN code; and an independent numpy
 *                   float32 evaluation of the reference's step order.
 *   gated_quant_fp8 closed forms: sigmoid(0) = 1/2 exactly, so act=sigmoid with a zero
 *                   gate quantises up/2; a gate of 30 has sigmoid 1 in f32, so silu
 *                   quantises bf16(30 * up); both through quant_act_fp8 (gate/up order,
 *                   the act switch and the bf16 narrowing fail them when wrong); plus a
 *                   numpy evaluation (float64 exp) on random and special gates, and NaN.
 *   rmsnorm_quant_fp8  integer-valued rows whose squares sum exactly in f32 in any order
 *                   (so the fold order drops out) against a numpy float32 evaluation;
 *                   the residual form equals the plain form on the written-back sum;
 *                   a power-of-two constant row has the closed form rs = 1/sqrt(c^2+eps).
 *                   The fold order itself is the reference kernel's, restated here and
 *                   met bit for bit by the device kernel's real shuffles.
 *   quant_dot       float64 brute force within the bound 2*K*2^-24*S + ulp_bf16;
 *                   single-nonzero closed forms; K=32 / K=128 single-group forms;
 *                   power-of-two scale exactness (a_scale linearity); 0xFF scale
 *                   poisons the element even when every code is zero; row / column
 *                   permutation equivariance (catches transposed operands).
 *   mxfp8 quantiser and mx8 x mxfp4 dot: same invariants, plus float64 brute force.
 *   f16 decode      all 65536 bit patterns vs numpy's float16 -> float32 (NaN as a class).
 *   logits_e4m3     float64 brute force within K*2^-24*S; every one of the 256 codes
 *                   through a one-hot x at unit scale (vs torch.float8_e4m3fn); a single
 *                   nonzero term is exact; power-of-two scales per 128-column block and per
 *                   row block (br = 128 against the same grid expanded to br = 1, bit for
 *                   bit); head-row permutation equivariance; a NaN code poisons its row.
 *   "parity unpinned" beyond these: no reference-held vectors exist for this path (the
 *   kbench packs are off-repo, tools/gate.sh:18-20), so bit-parity with libref itself on
 *   non-trivial inputs rests on the restatement below.
 */
#include "r3d_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* rad_fp8e4m3_to_f32 (as transcribed at src/r3d_gemm_mxfp4.hip:119-145 and
 * tools/probe_m4_entry.cpp:14-21): e4m3fn, bias 7, subnormal m*2^-9, S1111111 the only
 * NaN, no infinity. */
float r3d_ref_e4m3_to_f32(uint8_t b) {
    const uint32_t s = (uint32_t)(b >> 7) << 31;
    const uint32_t e = (b >> 3) & 0xFu, m = b & 0x7u;
    if (e == 0) {
        if (m == 0) return u2f(s);
        /* m * 2^-9: normalise the 3-bit field */
        uint32_t mm = m; int sh = 0;
        while (!(mm & 0x8u)) { mm <<= 1; ++sh; }
        return u2f(s | ((uint32_t)(127 - 6 - sh) << 23) | ((mm & 0x7u) << 20));
    }
    if (e == 0xF && m == 0x7) return u2f(s | 0x7FC00000u);
    return u2f(s | ((e - 7u + 127u) << 23) | (m << 20));
}

/* rad_fp4e2m1_to_f32 (src/r3d_gemm_mxfp4.hip:167-171, tools/probe_m4_entry.cpp:22):
 * 0, .5, 1, 1.5, 2, 3, 4, 6 with the sign bit 3; e2m1 has no NaN and no infinity. */
float r3d_ref_e2m1_to_f32(uint8_t nib) {
    static const float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
    const float v = mag[nib & 7u];
    return (nib & 8u) ? -v : v;
}

/* ref_common.h e8m0_to_f32 (tools/probe_m4_entry.cpp:85, src/r3d_mxfp4_q8x.h:17-37):
 * 0xFF is NaN, otherwise 2^(x-127); x = 0 is the f32 subnormal 2^-127. */
float r3d_ref_e8m0_to_f32(uint8_t x) {
    if (x == 0xFFu) return u2f(0x7FC00000u);
    if (x == 0u) return u2f(0x00400000u);
    return u2f((uint32_t)x << 23);
}

/* rad_f32_to_fp8e4m3 (transcribed at src/r3d_band.hip:61-87): round to nearest even,
 * subnormals by shift, saturate to +-448 (0x7E), NaN -> S1111111. */
uint8_t r3d_ref_f32_to_e4m3(float f) {
    const uint32_t u = f2u(f);
    const uint8_t s = (uint8_t)((u >> 24) & 0x80u);
    const uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint8_t)(s | 0x7Fu);
    if (a >= 0x43E00000u) return (uint8_t)(s | 0x7Eu);          /* >= 448 */
    const int e = (int)(a >> 23) - 127;
    uint32_t m = a & 0x7FFFFFu;
    if (e < -10) return s;                                       /* < 2^-10: to zero */
    if (e < -6) {                                                /* e4m3 subnormal */
        const int sh = -6 - e + 20;
        m |= 0x800000u;
        const uint32_t lo = m & ((1u << sh) - 1u);
        uint32_t q = m >> sh;
        const uint32_t half = 1u << (sh - 1);
        if (lo > half || (lo == half && (q & 1u))) ++q;
        return (uint8_t)(s | q);
    }
    uint32_t q = m >> 20;
    const uint32_t lo = m & 0xFFFFFu;
    if (lo > 0x80000u || (lo == 0x80000u && (q & 1u))) ++q;
    int ee = e + 7;
    if (q == 8u) { q = 0; ++ee; }
    if (ee > 15 || (ee == 15 && q >= 7u)) return (uint8_t)(s | 0x7Eu);
    return (uint8_t)(s | ((uint32_t)ee << 3) | q);
}

/* f32 -> bf16, round to nearest even, NaN kept quiet with its sign and upper payload
 * (src/r3d_gemm_mxfp4.hip:113-117, src/r3d_band.hip:52-56). */
uint16_t r3d_ref_f32_to_bf16(float f) {
    const uint32_t u = f2u(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

float r3d_ref_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

void r3d_ref_e4m3_to_f32_n(const uint8_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = r3d_ref_e4m3_to_f32(in[i]);
}
void r3d_ref_f32_to_e4m3_n(const float* in, uint8_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = r3d_ref_f32_to_e4m3(in[i]);
}
void r3d_ref_f32_to_bf16_n(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = r3d_ref_f32_to_bf16(in[i]);
}

void r3d_ref_mxfp4_dequant(const uint8_t* B, const uint8_t* BS, int64_t N, int64_t K,
                           int64_t bs_pitch, float* out) {
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k) {
            const uint8_t byte = B[n * (K / 2) + (k >> 1)];
            const uint8_t nib = (k & 1) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 0xF);
            out[n * K + k] = r3d_ref_e2m1_to_f32(nib) * r3d_ref_e8m0_to_f32(BS[n * bs_pitch + k / 32]);
        }
}

/* ref_gemm.h grid_block (as transcribed at src/r3d_gemm_mxfp4.hip:71-84): the block a
 * scale grid of `blocks` columns implies over `ext` -- the power of two whose ceiling
 * division gives exactly `blocks`, else the plain ceiling quotient. */
int64_t r3d_ref_grid_block(int64_t ext, int64_t blocks) {
    if (ext <= 0) return 1;
    if (blocks <= 1) return ext;
    const int64_t lo = (ext + blocks - 1) / blocks;
    int64_t p = 1;
    while (p < lo) p *= 2;
    return ((ext + p - 1) / p == blocks) ? p : lo;
}

static inline float ld_act(const void* x, int bf16, int64_t i) {
    return bf16 ? r3d_ref_bf16_to_f32(((const uint16_t*)x)[i]) : ((const float*)x)[i];
}

/* quant_act_fp8 (src/r3d_band.hip:11-14 for the rule, :117-153 for the kernel):
 * per (row, group): amax by strict '>' over fabsf (NaN never wins), scale =
 * amax * (1/448) or 1 for an all-zero group, codes = e4m3(clamp(x * (1/scale), +-448)). */
void r3d_ref_quant_act_fp8(const void* x, int x_is_bf16, int64_t M, int64_t K,
                           int64_t x_pitch, int64_t group, uint8_t* q, int64_t q_pitch,
                           float* scale, int64_t s_pitch) {
    const int64_t ng = (K + group - 1) / group;
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t g = 0; g < ng; ++g) {
            const int64_t k0 = g * group, k1 = (k0 + group < K) ? k0 + group : K;
            float amax = 0.0f;
            for (int64_t k = k0; k < k1; ++k) {
                const float a = fabsf(ld_act(x, x_is_bf16, m * x_pitch + k));
                if (a > amax) amax = a;
            }
            const float sc = amax > 0.0f ? amax * (1.0f / 448.0f) : 1.0f;
            scale[m * s_pitch + g] = sc;
            const float inv = 1.0f / sc;
            for (int64_t k = k0; k < k1; ++k) {
                float c = ld_act(x, x_is_bf16, m * x_pitch + k) * inv;
                if (c > 448.0f) c = 448.0f;
                if (c < -448.0f) c = -448.0f;
                q[m * q_pitch + k] = r3d_ref_f32_to_e4m3(c);
            }
        }
    }
}

/* gated_quant_fp8 (src/r3d_band.hip:155-201; the sigmoid at :46-47): per element
 * h = bf16(act(gate) * up) with sigmoid(x) = 1 / (1 + (float)exp((double)-x)) and
 * act(x) = silu ? x * sigmoid(x) : sigmoid(x); then quant_act_fp8's quantiser over each
 * group of h (h recomputed for the encode pass, as there); `out` (nullable) receives h's
 * bf16 bits.  gate_up rows: gate at [0, n), up at [n, 2n), row pitch gu_pitch. */
static inline float ref_gated_h(const void* gu, int bf16, int64_t i, int64_t n, int silu) {
    const float gt = ld_act(gu, bf16, i), up = ld_act(gu, bf16, i + n);
    const float e = (float)exp(-(double)gt);
    const float sg = 1.0f / (1.0f + e);
    const float t = silu ? gt * sg : sg;
    return r3d_ref_bf16_to_f32(r3d_ref_f32_to_bf16(t * up));
}

void r3d_ref_gated_quant_fp8(const void* gu, int gu_is_bf16, int64_t M, int64_t n,
                             int64_t gu_pitch, int64_t group, int silu, uint8_t* q,
                             int64_t q_pitch, float* scale, int64_t s_pitch, uint16_t* out,
                             int64_t out_pitch) {
    const int64_t ng = (n + group - 1) / group;
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t g = 0; g < ng; ++g) {
            const int64_t k0 = g * group, k1 = (k0 + group < n) ? k0 + group : n;
            float amax = 0.0f;
            for (int64_t k = k0; k < k1; ++k) {
                const float a = fabsf(ref_gated_h(gu, gu_is_bf16, m * gu_pitch + k, n, silu));
                if (a > amax) amax = a;
            }
            const float sc = amax > 0.0f ? amax * (1.0f / 448.0f) : 1.0f;
            scale[m * s_pitch + g] = sc;
            const float inv = 1.0f / sc;
            for (int64_t k = k0; k < k1; ++k) {
                const float h = ref_gated_h(gu, gu_is_bf16, m * gu_pitch + k, n, silu);
                if (out) out[m * out_pitch + k] = r3d_ref_f32_to_bf16(h);
                float c = h * inv;
                if (c > 448.0f) c = 448.0f;
                if (c < -448.0f) c = -448.0f;
                q[m * q_pitch + k] = r3d_ref_f32_to_e4m3(c);
            }
        }
    }
}

/* rmsnorm_quant_fp8 (src/r3d_more.hip:241-330), in the reference kernel's arithmetic
 * order: 256 lanes, lane t summing the squares of elements t, t+256, ... (multiply and add
 * separately rounded: that file is built with -ffp-contract=off); each 32-lane warp folded
 * by __shfl_down with offsets 16..1 (a lane whose source is past the warp adds its own
 * value, as the intrinsic returns it); the 8 warp sums added in order; then
 * rs = 1 / sqrtf(sum / n + eps).  With a residual, y = bf16(residual + x) is written back
 * first and squared.  h = bf16((src * rs) * (w + wadd)); `out` (nullable) gets h's bits;
 * quant_act_fp8's quantiser over each group of h. */
void r3d_ref_rmsnorm_quant_fp8(const uint16_t* x, int64_t M, int64_t n, int64_t x_pitch,
                               uint16_t* res, int64_t r_pitch, const void* w, int w_is_bf16,
                               int64_t group, float eps, float wadd, uint8_t* q,
                               int64_t q_pitch, float* scale, int64_t s_pitch, uint16_t* out,
                               int64_t out_pitch) {
    uint16_t* hs = (uint16_t*)malloc((size_t)n * sizeof(uint16_t));
    if (!hs) return;
    const int64_t ng = (n + group - 1) / group;
    for (int64_t m = 0; m < M; ++m) {
        const uint16_t* xr = x + m * x_pitch;
        uint16_t* rr = res ? res + m * r_pitch : 0;
        float lane[256];
        for (int t = 0; t < 256; ++t) {
            float ss = 0.0f;
            for (int64_t i = t; i < n; i += 256) {
                float v = r3d_ref_bf16_to_f32(xr[i]);
                if (rr) {
                    const uint16_t hb = r3d_ref_f32_to_bf16(r3d_ref_bf16_to_f32(rr[i]) + v);
                    rr[i] = hb;
                    hs[i] = hb;
                    v = r3d_ref_bf16_to_f32(hb);
                }
                const float sq = v * v;
                ss = ss + sq;
            }
            lane[t] = ss;
        }
        float warp[8];
        for (int wv = 0; wv < 8; ++wv) {
            float* l = lane + 32 * wv;
            for (int off = 16; off > 0; off >>= 1) {
                float nx[32];
                for (int i = 0; i < 32; ++i) nx[i] = l[i] + (i + off < 32 ? l[i + off] : l[i]);
                memcpy(l, nx, sizeof nx);
            }
            warp[wv] = l[0];
        }
        float r = warp[0];
        for (int k = 1; k < 8; ++k) r = r + warp[k];
        const float rs = 1.0f / sqrtf(r / (float)n + eps);
        for (int64_t i = 0; i < n; ++i) {
            const float src = rr ? r3d_ref_bf16_to_f32(hs[i]) : r3d_ref_bf16_to_f32(xr[i]);
            const float wv = (w_is_bf16 ? r3d_ref_bf16_to_f32(((const uint16_t*)w)[i])
                                        : ((const float*)w)[i]) + wadd;
            const float t1 = src * rs;
            hs[i] = r3d_ref_f32_to_bf16(t1 * wv);
            if (out) out[m * out_pitch + i] = hs[i];
        }
        r3d_ref_quant_act_fp8(hs, 1, 1, n, n, group, q + m * q_pitch, n, scale + m * s_pitch, ng);
    }
    free(hs);
}

#ifdef _OPENMP
#define R3D_SET_THREADS(n) int nth_ = (n) > 1 ? (n) : 1
#define R3D_PARALLEL_FOR _Pragma("omp parallel for schedule(static) num_threads(nth_)")
#else
#define R3D_SET_THREADS(n) (void)(n)
#define R3D_PARALLEL_FOR
#endif

/* quant_dot at mxfp4a8 (ref_gemm.h, as restated at src/r3d_gemm_mxfp4.hip:14-15 and
 * tools/probe_m4_entry.cpp:75-88): per 32-of-K group, an ascending f32 sum of exact
 * products, flushed as  acc += (sub * sa[m, k/128]) * 2^(x-127). */
void r3d_ref_quant_dot_mxfp4a8(const uint8_t* A, int64_t a_pitch, const float* AS,
                               int64_t as_pitch, const uint8_t* B, const uint8_t* BS,
                               int64_t bs_pitch, int64_t M, int64_t N, int64_t K,
                               uint16_t* Y, int64_t y_pitch, float* Yf, float* S,
                               int nthreads) {
    const int64_t ng = (K + 31) / 32;
    const int64_t bp = K / 2;
    R3D_SET_THREADS(nthreads);
    R3D_PARALLEL_FOR
    for (int64_t n = 0; n < N; ++n) {
        const uint8_t* brow = B + n * bp;
        const uint8_t* srow = BS + n * bs_pitch;
        for (int64_t m = 0; m < M; ++m) {
            const uint8_t* arow = A + m * a_pitch;
            float acc = 0.0f, mag = 0.0f;
            for (int64_t g = 0; g < ng; ++g) {
                const int64_t k0 = g * 32, k1 = (k0 + 32 < K) ? k0 + 32 : K;
                float sub = 0.0f, sab = 0.0f;
                for (int64_t k = k0; k < k1; ++k) {
                    const uint8_t byte = brow[k >> 1];
                    const uint8_t nib = (k & 1) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 0xF);
                    const float p = r3d_ref_e4m3_to_f32(arow[k]) * r3d_ref_e2m1_to_f32(nib);
                    sub = sub + p;
                    sab = sab + fabsf(p);
                }
                const float sa = AS[m * as_pitch + k0 / 128];
                const float sb = r3d_ref_e8m0_to_f32(srow[g]);
                acc = acc + (sub * sa) * sb;
                mag = mag + (sab * fabsf(sa)) * fabsf(sb);
            }
            Y[m * y_pitch + n] = r3d_ref_f32_to_bf16(acc);
            if (Yf) Yf[m * N + n] = acc;
            if (S) S[m * N + n] = mag;
        }
    }
}

/* quant_dot at fp8a8 (src/r3d_gemm_fp8a8.hip:9-15, tools/bench_fp8_skinny.cpp:399-420):
 * per 128-of-K group  acc += (sub * sa[m, g]) * bf16(sb[srow, g]),  srow = n / rblk. */
void r3d_ref_quant_dot_fp8a8(const uint8_t* A, int64_t a_pitch, const float* AS,
                             int64_t as_pitch, const uint8_t* B, int64_t b_pitch,
                             const uint16_t* BS, int64_t bs_pitch, int rblk,
                             int64_t M, int64_t N, int64_t K,
                             uint16_t* Y, int64_t y_pitch, float* Yf, float* S,
                             int nthreads) {
    const int64_t ng = (K + 127) / 128;
    R3D_SET_THREADS(nthreads);
    R3D_PARALLEL_FOR
    for (int64_t n = 0; n < N; ++n) {
        const uint8_t* brow = B + n * b_pitch;
        const uint16_t* srow = BS + (n / rblk) * bs_pitch;
        for (int64_t m = 0; m < M; ++m) {
            const uint8_t* arow = A + m * a_pitch;
            float acc = 0.0f, mag = 0.0f;
            for (int64_t g = 0; g < ng; ++g) {
                const int64_t k0 = g * 128, k1 = (k0 + 128 < K) ? k0 + 128 : K;
                float sub = 0.0f, sab = 0.0f;
                for (int64_t k = k0; k < k1; ++k) {
                    const float p = r3d_ref_e4m3_to_f32(arow[k]) * r3d_ref_e4m3_to_f32(brow[k]);
                    sub = sub + p;
                    sab = sab + fabsf(p);
                }
                const float sa = AS[m * as_pitch + g];
                const float sb = r3d_ref_bf16_to_f32(srow[g]);
                acc = acc + (sub * sa) * sb;
                mag = mag + (sab * fabsf(sa)) * fabsf(sb);
            }
            Y[m * y_pitch + n] = r3d_ref_f32_to_bf16(acc);
            if (Yf) Yf[m * N + n] = acc;
            if (S) S[m * N + n] = mag;
        }
    }
}

void r3d_ref_quant_act_mxfp8(const uint16_t* x, int64_t M, int64_t K, int64_t x_pitch,
                             uint8_t* q, int64_t q_pitch, uint8_t* sx, int64_t sx_pitch) {
    const int64_t ng = (K + 31) / 32;
    for (int64_t m = 0; m < M; ++m)
        for (int64_t g = 0; g < ng; ++g) {
            const int64_t k0 = g * 32, k1 = (k0 + 32 < K) ? k0 + 32 : K;
            float amax = 0.0f;
            for (int64_t k = k0; k < k1; ++k) {
                const float a = fabsf(r3d_ref_bf16_to_f32(x[m * x_pitch + k]));
                if (a > amax) amax = a;
            }
            int e = 0;
            if (amax > 0.0f && amax <= 3.4028235e38f) {
                /* least e with amax * 2^-e <= 448: amax = f * 2^ex, f in [0.5, 1) */
                int ex; const float f = frexpf(amax, &ex);
                e = (f > 0.875f) ? ex - 8 : ex - 9;
            }
            if (e < -127) e = -127;
            if (e > 127) e = 127;
            sx[m * sx_pitch + g] = (uint8_t)(e + 127);
            const float inv = ldexpf(1.0f, -e);
            for (int64_t k = k0; k < k1; ++k) {
                float c = r3d_ref_bf16_to_f32(x[m * x_pitch + k]) * inv;
                if (c > 448.0f) c = 448.0f;
                if (c < -448.0f) c = -448.0f;
                q[m * q_pitch + k] = r3d_ref_f32_to_e4m3(c);
            }
        }
}

void r3d_ref_dot_mx8_mxfp4(const uint8_t* A, int64_t a_pitch, const uint8_t* SX,
                           int64_t sx_pitch, const uint8_t* B, const uint8_t* BS,
                           int64_t bs_pitch, int64_t M, int64_t N, int64_t K,
                           uint16_t* Y, int64_t y_pitch, float* Yf, float* S,
                           int nthreads) {
    const int64_t ng = (K + 31) / 32;
    const int64_t bp = K / 2;
    R3D_SET_THREADS(nthreads);
    R3D_PARALLEL_FOR
    for (int64_t n = 0; n < N; ++n) {
        const uint8_t* brow = B + n * bp;
        const uint8_t* srow = BS + n * bs_pitch;
        for (int64_t m = 0; m < M; ++m) {
            const uint8_t* arow = A + m * a_pitch;
            float acc = 0.0f, mag = 0.0f;
            for (int64_t g = 0; g < ng; ++g) {
                const int64_t k0 = g * 32, k1 = (k0 + 32 < K) ? k0 + 32 : K;
                float sub = 0.0f, sab = 0.0f;
                for (int64_t k = k0; k < k1; ++k) {
                    const uint8_t byte = brow[k >> 1];
                    const uint8_t nib = (k & 1) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 0xF);
                    const float p = r3d_ref_e4m3_to_f32(arow[k]) * r3d_ref_e2m1_to_f32(nib);
                    sub = sub + p;
                    sab = sab + fabsf(p);
                }
                const float sa = r3d_ref_e8m0_to_f32(SX[m * sx_pitch + g]);
                const float sb = r3d_ref_e8m0_to_f32(srow[g]);
                acc = acc + (sub * sa) * sb;
                mag = mag + (sab * sa) * fabsf(sb);
            }
            Y[m * y_pitch + n] = r3d_ref_f32_to_bf16(acc);
            if (Yf) Yf[m * N + n] = acc;
            if (S) S[m * N + n] = mag;
        }
    }
}

void r3d_ref_group8_mag(int enc, const uint8_t* A, int64_t a_pitch, const float* AS,
                        int64_t as_pitch, const uint8_t* B, int64_t b_pitch, const void* BS,
                        int64_t bs_pitch, int rblk, int64_t M, int64_t N, int64_t K,
                        float* S8, int nthreads) {
    R3D_SET_THREADS(nthreads);
    R3D_PARALLEL_FOR
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t m = 0; m < M; ++m) {
            const uint8_t* arow = A + m * a_pitch;
            double tot = 0.0;
            for (int64_t k0 = 0; k0 < K; k0 += 8) {
                double mx = 0.0;
                for (int64_t k = k0; k < k0 + 8 && k < K; ++k) {
                    double w, sb;
                    if (enc != 1) {
                        const uint8_t byte = B[n * b_pitch + (k >> 1)];
                        const uint8_t nib = (k & 1) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 0xF);
                        w = r3d_ref_e2m1_to_f32(nib);
                        sb = r3d_ref_e8m0_to_f32(((const uint8_t*)BS)[n * bs_pitch + k / 32]);
                    } else {
                        w = r3d_ref_e4m3_to_f32(B[n * b_pitch + k]);
                        sb = r3d_ref_bf16_to_f32(((const uint16_t*)BS)[(n / rblk) * bs_pitch + k / 128]);
                    }
                    const double t = fabs(r3d_ref_e4m3_to_f32(arow[k]) * w * sb *
                                          AS[m * as_pitch + (enc == 2 ? k / 32 : k / 128)]);
                    if (t > mx) mx = t;           /* NaN never wins: the class check covers it */
                }
                tot += mx;
            }
            S8[m * N + n] = (float)tot;
        }
    }
}

float r3d_ref_f16_to_f32(uint16_t h) {
    const uint32_t sgn = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31u, m = h & 1023u;
    if (e == 31) return u2f(sgn | 0x7F800000u | (m << 13));          /* inf, NaN */
    if (e == 0) {
        const float v = (float)m * 0x1p-24f;                          /* m * 2^-24, exact */
        return sgn ? -v : v;
    }
    return u2f(sgn | ((e - 15u + 127u) << 23) | (m << 13));
}

static inline float ld_scale(const void* s, int sdt, int64_t i) {
    if (sdt == 2) return ((const float*)s)[i];
    const uint16_t v = ((const uint16_t*)s)[i];
    return sdt == 1 ? r3d_ref_f16_to_f32(v) : r3d_ref_bf16_to_f32(v);
}

/* logits_gemm over the joined e4m3 head (src/r3d_gemm_logits.hip:1-11 states the
 * reference's order; its kernel, :100-124, takes the same two steps per column): the
 * decoded code times the block scale, one f32 rounding, then one fused multiply-add into
 * the output's single f32 accumulator, over ascending k. */
void r3d_ref_logits_e4m3(const uint16_t* x, int64_t x_pitch, const uint8_t* codes,
                         const void* scale, int sdt, int64_t s_pitch, int br, int64_t M,
                         int64_t N, int64_t K, float* Y, int64_t y_pitch, float* S,
                         int nthreads) {
    R3D_SET_THREADS(nthreads);
    R3D_PARALLEL_FOR
    for (int64_t n = 0; n < N; ++n) {
        const uint8_t* crow = codes + n * K;
        const int64_t sbase = (n / br) * s_pitch;
        for (int64_t m = 0; m < M; ++m) {
            const uint16_t* xr = x + m * x_pitch;
            float acc = 0.0f, mag = 0.0f;
            for (int64_t k = 0; k < K; ++k) {
                const float cv = r3d_ref_e4m3_to_f32(crow[k]) * ld_scale(scale, sdt, sbase + k / 128);
                const float xv = r3d_ref_bf16_to_f32(xr[k]);
                acc = fmaf(xv, cv, acc);
                mag = mag + fabsf(xv * cv);
            }
            Y[m * y_pitch + n] = acc;
            if (S) S[m * N + n] = mag;
        }
    }
}

int r3d_ref_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
