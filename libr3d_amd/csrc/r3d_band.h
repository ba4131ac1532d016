/* r3d_band.h -- the activation producers on gfx950: quant_act_fp8, gated_quant_fp8 and
 * rmsnorm_quant_fp8 (below).  quant_act_fp8 is per-(row, group) symmetric e4m3 quantisation of a bf16 or f32
 * activation, plain row-major codes and an f32 dequant scale per group
 * (src/r3d_band.hip:117-153 of the reference):
 *     amax = max |x| over the group (NaN never wins; 0 when the group has none)
 *     sc   = amax > 0 ? amax * (1/448) : 1          (stored)
 *     q    = e4m3_rne(clamp(x * (1 / sc), +-448))   (NaN -> 0x7F with its sign)
 * One wave per (row, group): a first pass takes the maximum (v_max_f32, which skips NaN
 * like the reference's fmaxf reduction), a butterfly of lane shuffles spreads it, the
 * scale is a correctly rounded f32 multiply and divide (hipcc's default), and a second
 * pass encodes with v_cvt_pk_fp8_f32 (the same code as the oracle's encoder on every
 * clamped input; NaN fixed up).  With even groups, pitches and aligned bases each lane
 * moves two elements per pass (4 or 8 bytes in, 2 bytes out), else one.  The common case
 * (groups of 8..512 that tile the rows, aligned rows) takes the vector kernel below. */
#ifndef R3D_BAND_H
#define R3D_BAND_H

#include "r3d_device.h"

namespace r3d {

/* Four f32 (already inside +-448) -> four e4m3 codes, a in the low byte: two
 * v_cvt_pk_fp8_f32, then NaN inputs are set to 0x7F with their sign.  On MI355X this is
 * round-to-nearest-even e4m3 (the oracle's encoder) for every one of the 2^32 inputs after
 * the +-448 clamp (checked exhaustively on the device; the conversion alone differs only on
 * NaNs). */
__device__ __forceinline__ uint32_t r3d_e4m3x4_rne(float a, float b, float c, float d) {
    uint32_t w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, (int)w, true);
    const float x[4] = {a, b, c, d};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t nan = ((__float_as_uint(x[i]) >> 24) & 0x80u) | 0x7Fu;
        w = x[i] != x[i] ? (w & ~(0xFFu << (8 * i))) | (nan << (8 * i)) : w;
    }
    return w;
}

/* Two f32 (already inside +-448) -> two e4m3 codes in the low 16 bits, a in the low byte:
 * one v_cvt_pk_fp8_f32, then NaN inputs set to 0x7F with their sign (the conversion
 * differs from round-to-nearest-even e4m3 only on NaN; checked on all 2^32 inputs). */
__device__ __forceinline__ uint32_t r3d_e4m3x2_rne(float a, float b) {
    uint32_t w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xFFFFu;
    const uint32_t na = ((__float_as_uint(a) >> 24) & 0x80u) | 0x7Fu;
    const uint32_t nb = ((__float_as_uint(b) >> 24) & 0x80u) | 0x7Fu;
    w = a != a ? (w & 0xFF00u) | na : w;
    w = b != b ? (w & 0x00FFu) | (nb << 8) : w;
    return w;
}

template <bool BF16>
__device__ __forceinline__ float r3d_band_ld(const uint8_t* x, int64_t i) {
    if (BF16) return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(x)[i] << 16);
    return reinterpret_cast<const float*>(x)[i];
}

__device__ __forceinline__ float r3d_band_clamp448(float c) {
    if (c > 448.0f) c = 448.0f;                /* NaN passes both tests unchanged */
    if (c < -448.0f) c = -448.0f;
    return c;
}

/* items = rows * ngrp; 4 waves per workgroup, one item each.  x_pitch / q_pitch in
 * elements (0: every row reads / writes row 0, a rank-1 operand), s_pitch in floats. */
template <bool BF16, bool PAIR>
__global__ __launch_bounds__(256) void quant_act_fp8_kernel(
    const uint8_t* __restrict__ x, int64_t x_pitch, uint8_t* __restrict__ q, int64_t q_pitch,
    float* __restrict__ sc, int64_t s_pitch, int64_t n, int64_t g, int64_t ngrp, int64_t items) {
    const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= items) return;                            /* wave-uniform */
    const int lane = threadIdx.x & 63;
    const int64_t row = item / ngrp, gi = item - row * ngrp;
    const int64_t k0 = gi * g;
    const int64_t len = n - k0 < g ? n - k0 : g;
    const int64_t xb = row * x_pitch + k0;                /* element index of the group */
    constexpr int STEP = PAIR ? 128 : 64;
    const int64_t i0 = PAIR ? 2 * lane : lane;

    float amax = 0.0f;
    for (int64_t i = i0; i < len; i += STEP) {
        if (PAIR) {
            float v0, v1;
            if (BF16) {
                const uint32_t w = *reinterpret_cast<const uint32_t*>(x + 2 * (xb + i));
                v0 = __uint_as_float(w << 16);
                v1 = __uint_as_float(w & 0xFFFF0000u);
            } else {
                const float2 w = *reinterpret_cast<const float2*>(x + 4 * (xb + i));
                v0 = w.x;
                v1 = w.y;
            }
            amax = fmaxf(amax, fmaxf(fabsf(v0), fabsf(v1)));
        } else {
            amax = fmaxf(amax, fabsf(r3d_band_ld<BF16>(x, xb + i)));
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    const float s = amax > 0.0f ? amax * (1.0f / 448.0f) : 1.0f;
    if (lane == 0) sc[row * s_pitch + gi] = s;
    const float inv = 1.0f / s;

    uint8_t* qr = q + row * q_pitch + k0;
    for (int64_t i = i0; i < len; i += STEP) {
        if (PAIR) {
            float v0, v1;
            if (BF16) {
                const uint32_t w = *reinterpret_cast<const uint32_t*>(x + 2 * (xb + i));
                v0 = __uint_as_float(w << 16);
                v1 = __uint_as_float(w & 0xFFFF0000u);
            } else {
                const float2 w = *reinterpret_cast<const float2*>(x + 4 * (xb + i));
                v0 = w.x;
                v1 = w.y;
            }
            const uint32_t c = r3d_e4m3x2_rne(r3d_band_clamp448(v0 * inv),
                                              r3d_band_clamp448(v1 * inv));
            *reinterpret_cast<uint16_t*>(qr + i) = (uint16_t)c;
        } else {
            const float v = r3d_band_ld<BF16>(x, xb + i);
            qr[i] = (uint8_t)r3d_e4m3x2_rne(r3d_band_clamp448(v * inv), 0.0f);
        }
    }
}

/* Vector path: one workgroup per row, each thread 8 consecutive elements (one chunk) per
 * pass, its U chunks 256 chunks apart loaded before the first is used; the L = group / 8
 * lanes of a group (a power of two <= 64, so groups never straddle a wave) take the
 * maximum by log2(L) xor-shuffles.  Needs group % 8 == 0, n % group == 0, 16-byte aligned
 * x rows and 8-byte aligned q rows (the launch checks). */
constexpr int kQaU = 4;

template <bool BF16, int L>
__global__ __launch_bounds__(256) void quant_act_fp8_vec_kernel(
    const uint8_t* __restrict__ x, int64_t x_pitch, uint8_t* __restrict__ q, int64_t q_pitch,
    float* __restrict__ sc, int64_t s_pitch, int64_t n) {
    const int64_t row = blockIdx.x;
    const int64_t chunks = n >> 3;
    const uint8_t* xr = x + row * x_pitch * (BF16 ? 2 : 4);
    uint8_t* qr = q + row * q_pitch;
    float* sr = sc + row * s_pitch;
    for (int64_t c0 = threadIdx.x; c0 - threadIdx.x < chunks; c0 += 256 * kQaU) {
        float v[kQaU][8];
#pragma unroll
        for (int u = 0; u < kQaU; ++u) {
            /* a thread past the row's end re-reads its last chunk: the lanes of a group
             * leave the shuffles together, and nothing of it is stored */
            const int64_t c = c0 + 256 * u < chunks ? c0 + 256 * u : chunks - 1;
            if (BF16) {
                const r3d_i32x4 w = *reinterpret_cast<const r3d_i32x4*>(xr + 16 * c);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    v[u][2 * i] = __uint_as_float((uint32_t)w[i] << 16);
                    v[u][2 * i + 1] = __uint_as_float((uint32_t)w[i] & 0xFFFF0000u);
                }
            } else {
                const float4 a = *reinterpret_cast<const float4*>(xr + 32 * c);
                const float4 b = *reinterpret_cast<const float4*>(xr + 32 * c + 16);
                v[u][0] = a.x; v[u][1] = a.y; v[u][2] = a.z; v[u][3] = a.w;
                v[u][4] = b.x; v[u][5] = b.y; v[u][6] = b.z; v[u][7] = b.w;
            }
        }
#pragma unroll
        for (int u = 0; u < kQaU; ++u) {
            const int64_t c = c0 + 256 * u;
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[u][i]));
#pragma unroll
            for (int off = L / 2; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
            if (c >= chunks) continue;
            const float s = amax > 0.0f ? amax * (1.0f / 448.0f) : 1.0f;
            const float inv = 1.0f / s;
            if ((c & (L - 1)) == 0) sr[c / L] = s;
            float cv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) cv[i] = r3d_band_clamp448(v[u][i] * inv);
            const uint32_t lo = r3d_e4m3x4_rne(cv[0], cv[1], cv[2], cv[3]);
            const uint32_t hi = r3d_e4m3x4_rne(cv[4], cv[5], cv[6], cv[7]);
            *reinterpret_cast<uint2*>(qr + 8 * c) = make_uint2(lo, hi);
        }
    }
}

/* Few rows (decode): the same quantiser with one 8-element chunk per lane on a
 * (ceil(chunks / 256), rows) grid, so a row spreads over workgroups instead of one
 * workgroup walking it. */
template <bool BF16, int L>
__global__ __launch_bounds__(256) void quant_act_fp8_spread_kernel(
    const uint8_t* __restrict__ x, int64_t x_pitch, uint8_t* __restrict__ q, int64_t q_pitch,
    float* __restrict__ sc, int64_t s_pitch, int64_t n) {
    const int64_t row = blockIdx.y;
    const int64_t chunks = n >> 3;
    const uint8_t* xr = x + row * x_pitch * (BF16 ? 2 : 4);
    const int64_t c0 = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t c = c0 < chunks ? c0 : chunks - 1;   /* past the end: re-read, store nothing */
    float v[8];
    if (BF16) {
        const r3d_i32x4 w = *reinterpret_cast<const r3d_i32x4*>(xr + 16 * c);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = __uint_as_float((uint32_t)w[i] << 16);
            v[2 * i + 1] = __uint_as_float((uint32_t)w[i] & 0xFFFF0000u);
        }
    } else {
        const float4 a = *reinterpret_cast<const float4*>(xr + 32 * c);
        const float4 b = *reinterpret_cast<const float4*>(xr + 32 * c + 16);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
#pragma unroll
    for (int off = L / 2; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    if (c0 >= chunks) return;
    const float s = amax > 0.0f ? amax * (1.0f / 448.0f) : 1.0f;
    const float inv = 1.0f / s;
    if ((c & (L - 1)) == 0) sc[row * s_pitch + c / L] = s;
    float cv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) cv[i] = r3d_band_clamp448(v[i] * inv);
    *reinterpret_cast<uint2*>(q + row * q_pitch + 8 * c) =
        make_uint2(r3d_e4m3x4_rne(cv[0], cv[1], cv[2], cv[3]),
                   r3d_e4m3x4_rne(cv[4], cv[5], cv[6], cv[7]));
}

/* ---- gated_quant_fp8 (src/r3d_band.hip:155-201 of the reference): per element
 *     h = bf16(act(gate) * up),  act(x) = silu ? x * sigmoid(x) : sigmoid(x)
 *     sigmoid(x) = 1 / (1 + f32(exp_f64(-x)))        (exp in double, narrowed once)
 * with bf16() round-to-nearest-even (a NaN keeps its sign and top payload bits, quieted),
 * then quant_act_fp8's quantiser over each group of h.  The optional gated output is h
 * (bf16, exact) or h widened (f32). */
__device__ __forceinline__ uint32_t r3d_band_bf16_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float r3d_gated_h(float gt, float up, int silu) {
    const float e = (float)exp(-(double)gt);
    const float sg = 1.0f / (1.0f + e);
    const float t = silu ? gt * sg : sg;
    return __uint_as_float(r3d_band_bf16_bits(t * up) << 16);
}

/* One wave per (row, group), two passes (the gated value is recomputed for the encode pass:
 * the same instructions on the same inputs, so the same bits).  Pitches in elements; ob is
 * null when the gated output is not asked for. */
template <bool BF16>
__global__ __launch_bounds__(256) void gated_quant_fp8_kernel(
    const uint8_t* __restrict__ gu, int64_t gu_pitch, uint8_t* __restrict__ q, int64_t q_pitch,
    float* __restrict__ sc, int64_t s_pitch, uint8_t* __restrict__ ob, int ob_bf16,
    int64_t ob_pitch, int64_t n, int64_t g, int64_t ngrp, int64_t items, int silu) {
    const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= items) return;                            /* wave-uniform */
    const int lane = threadIdx.x & 63;
    const int64_t row = item / ngrp, gi = item - row * ngrp;
    const int64_t k0 = gi * g;
    const int64_t len = n - k0 < g ? n - k0 : g;
    const int64_t gb = row * gu_pitch + k0;
    float amax = 0.0f;
    for (int64_t i = lane; i < len; i += 64) {
        const float h = r3d_gated_h(r3d_band_ld<BF16>(gu, gb + i), r3d_band_ld<BF16>(gu, gb + n + i),
                                    silu);
        amax = fmaxf(amax, fabsf(h));
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    const float s = amax > 0.0f ? amax * (1.0f / 448.0f) : 1.0f;
    if (lane == 0) sc[row * s_pitch + gi] = s;
    const float inv = 1.0f / s;
    for (int64_t i = lane; i < len; i += 64) {
        const float h = r3d_gated_h(r3d_band_ld<BF16>(gu, gb + i), r3d_band_ld<BF16>(gu, gb + n + i),
                                    silu);
        if (ob) {
            if (ob_bf16)
                reinterpret_cast<uint16_t*>(ob)[row * ob_pitch + k0 + i] =
                    (uint16_t)(__float_as_uint(h) >> 16);
            else
                reinterpret_cast<float*>(ob)[row * ob_pitch + k0 + i] = h;
        }
        q[row * q_pitch + k0 + i] = (uint8_t)r3d_e4m3x2_rne(r3d_band_clamp448(h * inv), 0.0f);
    }
}

/* Groups of 8..512 tiling the rows (n % g == 0), aligned operands: grid (ceil(chunks / 256),
 * rows), one 8-element chunk per lane (16-byte gate and up loads at bf16) -- the exp in
 * double makes this ALU-heavy, so a row spreads over workgroups -- with L = g / 8 lanes per
 * group reducing the maximum by xor-shuffles; codes leave 8 bytes per lane, the gated
 * output 16 (bf16) or 32 (f32). */
template <bool BF16, int L>
__global__ __launch_bounds__(256) void gated_quant_fp8_vec_kernel(
    const uint8_t* __restrict__ gu, int64_t gu_pitch, uint8_t* __restrict__ q, int64_t q_pitch,
    float* __restrict__ sc, int64_t s_pitch, uint8_t* __restrict__ ob, int ob_bf16,
    int64_t ob_pitch, int64_t n, int silu) {
    constexpr int EB = BF16 ? 2 : 4;
    const int64_t row = blockIdx.y;
    const int64_t chunks = n >> 3;
    const uint8_t* gr = gu + row * gu_pitch * EB;
    const uint8_t* ur = gr + n * EB;
    /* a lane past the row's end re-reads its last chunk (its group's lanes leave the
     * shuffles together) and stores nothing */
    const int64_t c0 = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t c = c0 < chunks ? c0 : chunks - 1;
    float gv[8], uv[8];
    if (BF16) {
        const r3d_i32x4 a = *reinterpret_cast<const r3d_i32x4*>(gr + 16 * c);
        const r3d_i32x4 b = *reinterpret_cast<const r3d_i32x4*>(ur + 16 * c);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            gv[2 * i] = __uint_as_float((uint32_t)a[i] << 16);
            gv[2 * i + 1] = __uint_as_float((uint32_t)a[i] & 0xFFFF0000u);
            uv[2 * i] = __uint_as_float((uint32_t)b[i] << 16);
            uv[2 * i + 1] = __uint_as_float((uint32_t)b[i] & 0xFFFF0000u);
        }
    } else {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float4 a = *reinterpret_cast<const float4*>(gr + 32 * c + 16 * h);
            const float4 b = *reinterpret_cast<const float4*>(ur + 32 * c + 16 * h);
            gv[4 * h] = a.x; gv[4 * h + 1] = a.y; gv[4 * h + 2] = a.z; gv[4 * h + 3] = a.w;
            uv[4 * h] = b.x; uv[4 * h + 1] = b.y; uv[4 * h + 2] = b.z; uv[4 * h + 3] = b.w;
        }
    }
    float h[8];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        h[i] = r3d_gated_h(gv[i], uv[i], silu);
        amax = fmaxf(amax, fabsf(h[i]));
    }
#pragma unroll
    for (int off = L / 2; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    if (c0 >= chunks) return;
    const float s = amax > 0.0f ? amax * (1.0f / 448.0f) : 1.0f;
    const float inv = 1.0f / s;
    if ((c & (L - 1)) == 0) sc[row * s_pitch + c / L] = s;
    float cv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) cv[i] = r3d_band_clamp448(h[i] * inv);
    *reinterpret_cast<uint2*>(q + row * q_pitch + 8 * c) =
        make_uint2(r3d_e4m3x4_rne(cv[0], cv[1], cv[2], cv[3]),
                   r3d_e4m3x4_rne(cv[4], cv[5], cv[6], cv[7]));
    if (ob) {
        if (ob_bf16) {
            r3d_i32x4 o;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                o[i] = (int)((__float_as_uint(h[2 * i]) >> 16) |
                             (__float_as_uint(h[2 * i + 1]) & 0xFFFF0000u));
            *reinterpret_cast<r3d_i32x4*>(ob + 2 * (row * ob_pitch + 8 * c)) = o;
        } else {
            float* of = reinterpret_cast<float*>(ob) + row * ob_pitch + 8 * c;
            *reinterpret_cast<float4*>(of) = make_float4(h[0], h[1], h[2], h[3]);
            *reinterpret_cast<float4*>(of + 4) = make_float4(h[4], h[5], h[6], h[7]);
        }
    }
}

/* ---- rmsnorm_quant_fp8 (src/r3d_more.hip:241-330 of the reference), one workgroup of 256
 * lanes per row, the row's bf16 values staged in LDS:
 *   0. stage the row: with a residual, y = bf16(residual + x) is stored back and staged;
 *      else x is staged (16-byte loads and stores when VEC, else element by element --
 *      every load independent, so all are in flight together).
 *   1. lane t sums the squares of staged elements t, t + 256, ... in that order (separately
 *      rounded multiply and add: the reference builds this file without contraction); the
 *      256 partials then fold exactly as the reference's 32-lane warps do -- a shuffle-down
 *      tree inside each 32-lane half (offsets 16, 8, 4, 2, 1), and the eight half sums added
 *      in order -- so the sum is bit-identical.
 *   2. rs = 1 / sqrt(sum / n + eps);  h = bf16((src * rs) * (w + wadd)), the normed value
 *      out_bf16 carries and the quantiser sees (elementwise, any lane order).
 *   3. quant_act_fp8's quantiser over each group of h: VQ -- groups of 8..512 tiling the
 *      row -- L = g / 8 lanes per group, 8 values a lane, xor-shuffle maximum; else one wave
 *      per group.  The maximum is order-free. */
template <bool WBF16, bool VEC, int L>
__global__ __launch_bounds__(256) void rmsnorm_quant_fp8_kernel(
    const uint16_t* __restrict__ x, int64_t x_pitch, uint16_t* __restrict__ res, int64_t r_pitch,
    const uint8_t* __restrict__ w, uint8_t* __restrict__ q, int64_t q_pitch,
    float* __restrict__ sc, int64_t s_pitch, uint8_t* __restrict__ ob, int ob_bf16,
    int64_t ob_pitch, int n, int g, int ngrp, float eps, float wadd) {
    extern __shared__ __attribute__((aligned(16))) uint16_t s_h[];
    __shared__ float s_part[8];
    __shared__ float s_rs;
    const int t = threadIdx.x;
    const int64_t row = blockIdx.x;
    const uint16_t* xr = x + row * x_pitch;
    uint16_t* rr = res ? res + row * r_pitch : nullptr;
    auto bf = [](uint32_t b) { return __uint_as_float(b << 16); };
    constexpr int U = 4;                        /* chunks a lane loads before using any */
    const int nc = n >> 3;
    if (VEC) {
        for (int c0 = t; c0 < nc; c0 += 256 * U) {
            r3d_i32x4 v[U], a[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int c = c0 + 256 * u < nc ? c0 + 256 * u : nc - 1;
                v[u] = *reinterpret_cast<const r3d_i32x4*>(xr + 8 * c);
                if (rr) a[u] = *reinterpret_cast<const r3d_i32x4*>(rr + 8 * c);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int c = c0 + 256 * u;
                if (c >= nc) break;
                if (rr) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t lo = r3d_band_bf16_bits(__fadd_rn(
                            bf((uint32_t)a[u][i] & 0xFFFFu), bf((uint32_t)v[u][i] & 0xFFFFu)));
                        const uint32_t hi = r3d_band_bf16_bits(__fadd_rn(
                            bf((uint32_t)a[u][i] >> 16), bf((uint32_t)v[u][i] >> 16)));
                        v[u][i] = (int)(lo | (hi << 16));
                    }
                    *reinterpret_cast<r3d_i32x4*>(rr + 8 * c) = v[u];
                }
                *reinterpret_cast<r3d_i32x4*>(s_h + 8 * c) = v[u];
            }
        }
    } else {
#pragma unroll 4
        for (int i = t; i < n; i += 256) {
            uint32_t hb = xr[i];
            if (rr) {
                hb = r3d_band_bf16_bits(__fadd_rn(bf(rr[i]), bf(hb)));
                rr[i] = (uint16_t)hb;
            }
            s_h[i] = (uint16_t)hb;
        }
    }
    __syncthreads();
    float ss = 0.0f;
    for (int i = t; i < n; i += 256) {
        const float v = bf(s_h[i]);
        ss = __fadd_rn(ss, __fmul_rn(v, v));
    }
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) ss = __fadd_rn(ss, __shfl_down(ss, off, 32));
    if ((t & 31) == 0) s_part[t >> 5] = ss;
    __syncthreads();
    if (t == 0) {
        float r = s_part[0];
        for (int k = 1; k < 8; ++k) r = __fadd_rn(r, s_part[k]);
        s_rs = 1.0f / sqrtf(__fadd_rn(r / (float)n, eps));
    }
    __syncthreads();
    const float rs = s_rs;
    auto wval = [&](int i) {
        return __fadd_rn(WBF16 ? bf(reinterpret_cast<const uint16_t*>(w)[i])
                               : reinterpret_cast<const float*>(w)[i], wadd);
    };
    if (VEC) {
        for (int c0 = t; c0 < nc; c0 += 256 * U) {
            float wv[U][8];
#pragma unroll
            for (int u = 0; u < U; ++u) {               /* the batch's w loads first */
                const int c = c0 + 256 * u < nc ? c0 + 256 * u : nc - 1;
                if (WBF16) {
                    const r3d_i32x4 a = *reinterpret_cast<const r3d_i32x4*>(w + 16 * c);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        wv[u][2 * i] = bf((uint32_t)a[i] & 0xFFFFu);
                        wv[u][2 * i + 1] = bf((uint32_t)a[i] >> 16);
                    }
                } else {
                    const float4 a = *reinterpret_cast<const float4*>(w + 32 * c);
                    const float4 b = *reinterpret_cast<const float4*>(w + 32 * c + 16);
                    wv[u][0] = a.x; wv[u][1] = a.y; wv[u][2] = a.z; wv[u][3] = a.w;
                    wv[u][4] = b.x; wv[u][5] = b.y; wv[u][6] = b.z; wv[u][7] = b.w;
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int c = c0 + 256 * u;
                if (c >= nc) break;
                const r3d_i32x4 v = *reinterpret_cast<const r3d_i32x4*>(s_h + 8 * c);
                r3d_i32x4 o;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t lo = r3d_band_bf16_bits(__fmul_rn(
                        __fmul_rn(bf((uint32_t)v[i] & 0xFFFFu), rs), __fadd_rn(wv[u][2 * i], wadd)));
                    const uint32_t hi = r3d_band_bf16_bits(__fmul_rn(
                        __fmul_rn(bf((uint32_t)v[i] >> 16), rs), __fadd_rn(wv[u][2 * i + 1], wadd)));
                    o[i] = (int)(lo | (hi << 16));
                }
                if (ob) {
                    if (ob_bf16) {
                        *reinterpret_cast<r3d_i32x4*>(ob + 2 * (row * ob_pitch + 8 * c)) = o;
                    } else {
                        float* of = reinterpret_cast<float*>(ob) + row * ob_pitch + 8 * c;
                        *reinterpret_cast<float4*>(of) =
                            make_float4(bf((uint32_t)o[0] & 0xFFFFu), bf((uint32_t)o[0] >> 16),
                                        bf((uint32_t)o[1] & 0xFFFFu), bf((uint32_t)o[1] >> 16));
                        *reinterpret_cast<float4*>(of + 4) =
                            make_float4(bf((uint32_t)o[2] & 0xFFFFu), bf((uint32_t)o[2] >> 16),
                                        bf((uint32_t)o[3] & 0xFFFFu), bf((uint32_t)o[3] >> 16));
                    }
                }
                *reinterpret_cast<r3d_i32x4*>(s_h + 8 * c) = o;
            }
        }
    } else {
        for (int i = t; i < n; i += 256) {
            const uint32_t h = r3d_band_bf16_bits(__fmul_rn(__fmul_rn(bf(s_h[i]), rs), wval(i)));
            if (ob) {
                if (ob_bf16) reinterpret_cast<uint16_t*>(ob)[row * ob_pitch + i] = (uint16_t)h;
                else reinterpret_cast<float*>(ob)[row * ob_pitch + i] = bf(h);
            }
            s_h[i] = (uint16_t)h;
        }
    }
    __syncthreads();
    if (L > 0) {
        /* groups of 8 L values tiling the row: L lanes a group, 8 values a lane */
        for (int c0 = t; c0 - t < nc; c0 += 256) {
            const int c = c0 < nc ? c0 : nc - 1;
            const r3d_i32x4 v = *reinterpret_cast<const r3d_i32x4*>(s_h + 8 * c);
            float h[8];
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                h[2 * i] = bf((uint32_t)v[i] & 0xFFFFu);
                h[2 * i + 1] = bf((uint32_t)v[i] >> 16);
                amax = fmaxf(amax, fmaxf(fabsf(h[2 * i]), fabsf(h[2 * i + 1])));
            }
#pragma unroll
            for (int off = L / 2; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
            if (c0 >= nc) continue;
            const float s = amax > 0.0f ? amax * (1.0f / 448.0f) : 1.0f;
            if ((c & (L - 1)) == 0) sc[row * s_pitch + c / L] = s;
            const float inv = 1.0f / s;
            float cv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) cv[i] = r3d_band_clamp448(h[i] * inv);
            *reinterpret_cast<uint2*>(q + row * q_pitch + 8 * c) =
                make_uint2(r3d_e4m3x4_rne(cv[0], cv[1], cv[2], cv[3]),
                           r3d_e4m3x4_rne(cv[4], cv[5], cv[6], cv[7]));
        }
    } else {
        const int wave = t >> 6, lane = t & 63;
        for (int gi = wave; gi < ngrp; gi += 4) {             /* wave-uniform */
            const int k0 = gi * g, len = n - k0 < g ? n - k0 : g;
            float amax = 0.0f;
            for (int i = lane; i < len; i += 64) amax = fmaxf(amax, fabsf(bf(s_h[k0 + i])));
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
            const float s = amax > 0.0f ? amax * (1.0f / 448.0f) : 1.0f;
            if (lane == 0) sc[row * s_pitch + gi] = s;
            const float inv = 1.0f / s;
            for (int i = lane; i < len; i += 64)
                q[row * q_pitch + k0 + i] = (uint8_t)r3d_e4m3x2_rne(
                    r3d_band_clamp448(bf(s_h[k0 + i]) * inv), 0.0f);
        }
    }
}

}  // namespace r3d

#endif /* R3D_BAND_H */
