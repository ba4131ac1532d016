/* r3d_band.h -- the quant_act_fp8 producer on gfx950: per-(row, group) symmetric e4m3
 * quantisation of a bf16 or f32 activation, plain row-major codes and an f32 dequant
 * scale per group (src/r3d_band.hip:117-153 of the reference):
 *     amax = max |x| over the group (NaN never wins; 0 when the group has none)
 *     sc   = amax > 0 ? amax * (1/448) : 1          (stored)
 *     q    = e4m3_rne(clamp(x * (1 / sc), +-448))   (NaN -> 0x7F with its sign)
 * One wave per (row, group): a first pass takes the maximum (v_max_f32, which skips NaN
 * like the reference's fmaxf reduction), a butterfly of lane shuffles spreads it, the
 * scale is a correctly rounded f32 multiply and divide (hipcc's default), and a second
 * pass encodes with v_cvt_pk_fp8_f32 (the same code as the oracle's encoder on every
 * clamped input; NaN fixed up).  With even groups, pitches and aligned bases each lane
 * moves two elements per pass (4 or 8 bytes in, 2 bytes out), else one. */
#ifndef R3D_BAND_H
#define R3D_BAND_H

#include "r3d_device.h"

namespace r3d {

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

}  // namespace r3d

#endif /* R3D_BAND_H */
