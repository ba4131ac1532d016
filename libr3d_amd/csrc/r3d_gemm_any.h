/* r3d_gemm_any.h -- the gemm_nt_q arm for operands at any alignment.
 *
 * The fast arms stream A and B with 16-byte loads (into registers or straight into LDS),
 * so they need 16-byte aligned bases and pitches.  The reference's rows take any
 * alignment: its tile rows read bytes ("anything odd rides the tile",
 * src/r3d_gemm_fp8a8.hip:985-990,1090-1095; src/r3d_gemm_mxfp4.hip:1521-1582).  This
 * kernel takes every operand at any byte address and any pitch: each 16-byte operand
 * piece is assembled from five dword loads at 4-byte aligned offsets and funnel-shifted
 * into place (v_alignbit), and scale elements the same way from two.  A dword load
 * touches only dwords that hold at least one byte of the operand (the buffer's record
 * count ends at the dword holding the operand's last byte, so a dword past it reads 0
 * without touching memory), so no access is misaligned and none leaves the operand.
 *
 * The arithmetic is the prefill tile's, per 128-wide K step and 16 x 16 output fragment:
 * one v_mfma_scale_f32_16x16x128_f8f6f4 with weights as source A and activations as
 * source B (r3d_device.h layouts), and libref's flush -- mxfp4a8: the E8M0 weight scales
 * in the MFMA, acc += D * a_scale; fp8a8: acc += (D * a_scale) * b_scale; mxfp8
 * activations (mxfp4a16): both E8M0 scales in the MFMA, accumulating in place.
 *
 * Geometry: a wave owns 32 weight rows (two fragments) x 16 TM tokens; a workgroup is 4
 * waves along N (128 weight rows).  Grid (ceil(N / 128), ceil(M / (16 TM))).
 */
#ifndef R3D_GEMM_ANY_H
#define R3D_GEMM_ANY_H

#include "r3d_device.h"
#include "r3d_prefill_layout.h"

namespace r3d {

constexpr uint32_t kAnyOob = 0x80000000u;     /* past every record count: reads 0 */

/* A buffer over an operand starting at any byte: the resource begins at the dword that
 * holds the first byte, d bytes before it. */
struct AnyBuf {
    __amdgpu_buffer_rsrc_t r;
    uint32_t d;
};

__device__ __forceinline__ AnyBuf any_buf(const void* p, int64_t bytes) {
    const uintptr_t u = reinterpret_cast<uintptr_t>(p);
    const uintptr_t b = u & ~(uintptr_t)3;
    AnyBuf o;
    o.d = (uint32_t)(u - b);
    o.r = r3d_rsrc(reinterpret_cast<const void*>(b), bytes > 0 ? (bytes + o.d + 3) & ~(int64_t)3 : 0);
    return o;
}

__device__ __forceinline__ uint32_t any_dw(const AnyBuf& b, uint32_t off) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(b.r, (int)off, 0, 0);
}

/* Four bytes at byte `o` of the operand (kAnyOob: zeros). */
__device__ __forceinline__ uint32_t any_ld4(const AnyBuf& b, uint32_t o) {
    const uint32_t x = o + b.d, f = x & ~3u;
    return __builtin_amdgcn_alignbit(any_dw(b, f + 4), any_dw(b, f), (x & 3u) * 8u);
}

/* Sixteen bytes at byte `o` of the operand (kAnyOob: zeros); al16: the operand's pieces
 * are 16-byte aligned, one dwordx4 load. */
__device__ __forceinline__ r3d_i32x4 any_ld16(const AnyBuf& b, uint32_t o, bool al16) {
    if (al16)
        return __builtin_bit_cast(r3d_i32x4,
                                  __builtin_amdgcn_raw_buffer_load_b128(b.r, (int)(o + b.d), 0, 0));
    const uint32_t x = o + b.d, f = x & ~3u, s = (x & 3u) * 8u;
    uint32_t w[5];
#pragma unroll
    for (int j = 0; j < 5; ++j) w[j] = any_dw(b, f + 4 * j);
    r3d_i32x4 v;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = (int)__builtin_amdgcn_alignbit(w[j + 1], w[j], s);
    return v;
}

__device__ __forceinline__ uint32_t any_ld1(const AnyBuf& b, uint32_t o) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(b.r, (int)(o + b.d), 0, 0);
}

/* The fp8 operand of one 128-wide step of a row at byte `o`: [16 kb, +16) and [64 + 16 kb,
 * +16). */
__device__ __forceinline__ r3d_i32x8 any_fp8_operand(const AnyBuf& b, uint32_t o, int kb,
                                                     bool al16, bool in) {
    const r3d_i32x4 lo = any_ld16(b, in ? o + 16 * kb : kAnyOob, al16);
    const r3d_i32x4 hi = any_ld16(b, in ? o + 64 + 16 * kb : kAnyOob, al16);
    return r3d_i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

template <int MODE, int TM>
__global__ __launch_bounds__(256) void gemm_any_kernel(
    const uint8_t* __restrict__ A, const void* __restrict__ AS, const uint8_t* __restrict__ B,
    const uint8_t* __restrict__ BS, uint16_t* __restrict__ Y, int M, int N, int steps, int rblk,
    int64_t a_pitch, int64_t as_pitch, int64_t b_pitch, int64_t bs_pitch, int64_t y_pitch) {
    constexpr bool F8 = MODE == PF_F8, MX8 = MODE == PF_MX8;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, q = lane >> 4;
    const int64_t n0 = (int64_t)blockIdx.x * 128 + 32 * wave;
    const int64_t m0 = (int64_t)blockIdx.y * 16 * TM;
    if (n0 >= N) return;                                /* whole wave: no barrier follows */
    const int nrows = N - n0 < 32 ? (int)(N - n0) : 32;
    const int mrows = M - m0 < 16 * TM ? (int)(M - m0) : 16 * TM;
    const int64_t K = (int64_t)steps * 128;
    const int64_t wrow = F8 ? K : K / 2;                /* weight bytes a row */

    const uint8_t* bp = B + n0 * b_pitch;
    const uint8_t* ap = A + m0 * a_pitch;
    const AnyBuf bw = any_buf(bp, (nrows - 1) * b_pitch + wrow);
    const AnyBuf ba = any_buf(ap, (mrows - 1) * a_pitch + K);
    const bool wal = ((reinterpret_cast<uintptr_t>(bp) | (uintptr_t)b_pitch) & 15) == 0;
    const bool aal = ((reinterpret_cast<uintptr_t>(ap) | (uintptr_t)a_pitch) & 15) == 0;
    /* weight scales: E8M0 bytes [row][K/32], or bf16 [row / rblk][K/128] */
    const int64_t srow0 = F8 ? n0 / rblk : n0;
    const int64_t srows = F8 ? (n0 + nrows - 1) / rblk - srow0 + 1 : nrows;
    const int64_t s_cols = F8 ? steps : 4 * (int64_t)steps;
    const int esz_b = F8 ? 2 : 1;
    const AnyBuf bsb = any_buf(BS + srow0 * bs_pitch * esz_b, ((srows - 1) * bs_pitch + s_cols) * esz_b);
    /* activation scales: f32 [token][K/128], or E8M0 bytes [token][K/32] */
    const int esz_a = MX8 ? 1 : 4;
    const int64_t a_cols = MX8 ? 4 * (int64_t)steps : steps;
    const AnyBuf asb = any_buf(reinterpret_cast<const uint8_t*>(AS) + m0 * as_pitch * esz_a,
                               ((mrows - 1) * as_pitch + a_cols) * esz_a);

    r3d_f32x4 acc[2][TM];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int u = 0; u < TM; ++u) acc[t][u] = r3d_f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    for (int s = 0; s < steps; ++s) {
        r3d_i32x8 w8[2];
        r3d_i32x4 w4[2];
        int ws[2];
        float sb[2][4];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int row = 16 * t + r16;
            const bool in = row < nrows;
            const uint32_t ro = (uint32_t)(row * b_pitch);
            if (F8) {
                w8[t] = any_fp8_operand(bw, ro + 128u * s, q, wal, in);
                /* the four weight rows 16 t + 4 q + i whose results this lane holds */
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int64_t n = n0 + 16 * t + 4 * q + i;
                    const uint32_t so = n < N ? (uint32_t)(((n / rblk - srow0) * bs_pitch + s) * 2)
                                              : kAnyOob;
                    sb[t][i] = __uint_as_float(any_ld4(bsb, so) << 16);
                }
            } else {
                w4[t] = any_ld16(bw, in ? ro + 64u * s + 16u * q : kAnyOob, wal);
                ws[t] = (int)any_ld1(bsb, in ? (uint32_t)(row * bs_pitch + 4 * s + q) : kAnyOob);
            }
        }
        r3d_i32x8 x8[TM];
        float sa[TM];
        int xs[TM];
#pragma unroll
        for (int u = 0; u < TM; ++u) {
            const int tok = 16 * u + r16;
            const bool in = tok < mrows;
            x8[u] = any_fp8_operand(ba, (uint32_t)(tok * a_pitch) + 128u * s, q, aal, in);
            if (MX8) {
                xs[u] = (int)any_ld1(asb, in ? (uint32_t)(tok * as_pitch + 4 * s + q) : kAnyOob);
            } else {
                sa[u] = __uint_as_float(any_ld4(asb, in ? (uint32_t)((tok * as_pitch + s) * 4)
                                                        : kAnyOob));
            }
        }
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int u = 0; u < TM; ++u) {
                if (MX8) {
                    acc[t][u] = r3d_mfma_fp4_fp8_acc(w4[t], ws[t], x8[u], xs[u], acc[t][u]);
                } else if (F8) {
                    const r3d_f32x4 d = r3d_mfma_fp8_fp8(w8[t], x8[u]);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[t][u][i] = acc[t][u][i] + (d[i] * sa[u]) * sb[t][i];
                } else {
                    const r3d_f32x4 d = r3d_mfma_fp4_fp8(w4[t], ws[t], x8[u], R3D_E8M0_ONE);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[t][u][i] = acc[t][u][i] + d[i] * sa[u];
                }
            }
    }
    /* lane holds D[16 t + 4 q + i][16 u + r16]: weight rows x tokens; 2-byte stores */
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int u = 0; u < TM; ++u) {
            asm volatile("" : "+v"(acc[t][u]));    /* no MFMA sinks into the store branches */
            const int tok = 16 * u + r16;
            if (tok >= mrows) continue;
            uint16_t* yp = Y + (m0 + tok) * y_pitch + n0 + 16 * t + 4 * q;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (16 * t + 4 * q + i < nrows) yp[i] = r3d_bf16_rne(acc[t][u][i]);
        }
}

}  // namespace r3d

#endif /* R3D_GEMM_ANY_H */
