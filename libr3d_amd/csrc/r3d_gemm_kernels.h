/* r3d_gemm_kernels.h -- gfx950 kernels of gemm_nt_q at mxfp4a8 and fp8a8.
 *
 * Both encodings compute  Y[m, n] = sum_g (sub_g * a_scale[m, g]) * b_scale[n, g]  with
 * the 128-of-K activation-scale group as the unit of work: one
 * v_mfma_scale_f32_16x16x128_f8f6f4 covers exactly one activation group, so its result
 * is scaled by a_scale in f32 and accumulated, as libref's quant_dot flushes per group
 * (src/r3d_gemm_mxfp4.hip:14-15, src/r3d_gemm_fp8a8.hip:9-15).  The mxfp4 weight scales
 * (E8M0, per 32 of K) ride the MFMA's own scale operand -- a power of two, applied
 * exactly -- so the e2m1 nibbles go from HBM to the matrix core with no VALU decode.
 * The fp8a8 weight scale (bf16, per 128 of K) is applied after a_scale, in the oracle's
 * (sub * sa) * sb order.
 *
 * Orientation: weights are MFMA source A (16 weight rows per operand), activations are
 * source B (16 activation rows), so D[n][m] lands with one activation row per lane
 * (lane%16) and four consecutive weight rows per lane (4*(lane/16) + i).
 */
#ifndef R3D_GEMM_KERNELS_H
#define R3D_GEMM_KERNELS_H

#include "r3d_device.h"
#include "r3d_plan.h"

namespace r3d {

/* ---------------------------------------------------------------- decode GEMV ------
 * One wave owns a 16-row weight tile and one contiguous chunk of its K steps; the
 * `chunks` waves of a tile sit in the same workgroup and fold their f32 partials through
 * LDS in chunk order (deterministic).  Weight bytes are read once, with non-temporal
 * 16-byte loads, PF steps ahead of use; activation rows m >= M load nothing (zeros),
 * weight rows n >= N clamp their loads to row N-1 and never store. */
template <int ENC, int MT, int PF>
__global__ __launch_bounds__(512) void gemv_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ AS,
    const uint8_t* __restrict__ B, const void* __restrict__ BSv,
    uint16_t* __restrict__ Y,
    int M, int N, int steps, int chunks, int rblk,
    int64_t a_pitch, int64_t as_pitch, int64_t b_pitch, int64_t bs_pitch, int64_t y_pitch) {
    __shared__ r3d_f32x4 red[8][64];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int waves = blockDim.x >> 6;
    const int tpb = waves / chunks;
    const int64_t tile = (int64_t)blockIdx.x * tpb + wave / chunks;
    const int c = wave % chunks;
    const int s0 = (int)((int64_t)steps * c / chunks);
    const int s1 = (int)((int64_t)steps * (c + 1) / chunks);

    const int q = lane >> 4;           /* K sub-block of this lane inside a step */
    const int li = lane & 15;          /* weight row (src A) / activation row (src B) */
    const int64_t n0 = tile * 16;
    int64_t nl = n0 + li;
    if (nl > N - 1) nl = N - 1;        /* dead rows and whole dead tiles clamp their loads */

    const bool a_live = li < M && li < MT;
    const uint8_t* wrow;
    const uint8_t* srow = nullptr;
    if (ENC == ENC_MXFP4A8) {
        wrow = B + nl * b_pitch + 16 * q;
        srow = reinterpret_cast<const uint8_t*>(BSv) + nl * bs_pitch + q;
    } else {
        wrow = B + nl * b_pitch;
    }
    const uint8_t* arow = A + (int64_t)(a_live ? li : 0) * a_pitch;
    const float* asrow = AS + (int64_t)(a_live ? li : 0) * as_pitch;

    /* fp8a8 weight scales: four weight rows per lane (rows 4q .. 4q+3 of the tile). */
    const uint16_t* sbrow[4] = {nullptr, nullptr, nullptr, nullptr};
    if (ENC == ENC_FP8A8) {
        const uint16_t* BS16 = reinterpret_cast<const uint16_t*>(BSv);
        for (int i = 0; i < 4; ++i) {
            int64_t nr = n0 + 4 * q + i;
            if (nr > N - 1) nr = N - 1;
            sbrow[i] = BS16 + (nr / rblk) * bs_pitch;
        }
    }

    r3d_f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};

    /* prefetch ring */
    r3d_i32x4 wq[PF];
    r3d_i32x8 w8[PF];
    int sc[PF];
    r3d_i32x8 av[PF];
    float sa[PF];
    float sb[PF][4];

    auto issue = [&](int u, int s) {
        if (ENC == ENC_MXFP4A8) {
            wq[u] = r3d_ld16_stream(wrow + 64 * (int64_t)s);
            sc[u] = srow[4 * (int64_t)s];
        } else {
            w8[u] = r3d_ld_fp8_operand_stream(wrow + 128 * (int64_t)s, q);
            for (int i = 0; i < 4; ++i) sb[u][i] = r3d_bf16_to_f32(sbrow[i][s]);
        }
        if (a_live) {
            av[u] = r3d_ld_fp8_operand(arow + 128 * (int64_t)s, q);
            sa[u] = asrow[s];
        } else {
            const r3d_i32x8 z = {0, 0, 0, 0, 0, 0, 0, 0};
            av[u] = z;
            sa[u] = 0.0f;
        }
    };

#pragma unroll
    for (int u = 0; u < PF; ++u)
        if (s0 + u < s1) issue(u, s0 + u);

    for (int s = s0; s < s1; s += PF) {
#pragma unroll
        for (int u = 0; u < PF; ++u) {
            const int ss = s + u;
            if (ss < s1) {
                r3d_f32x4 d;
                if (ENC == ENC_MXFP4A8) {
                    d = r3d_mfma_fp4_fp8(wq[u], sc[u], av[u], R3D_E8M0_ONE);
                    const float a_s = sa[u];
                    for (int i = 0; i < 4; ++i) acc[i] = acc[i] + d[i] * a_s;
                } else {
                    d = r3d_mfma_fp8_fp8(w8[u], av[u]);
                    const float a_s = sa[u];
                    for (int i = 0; i < 4; ++i) acc[i] = acc[i] + (d[i] * a_s) * sb[u][i];
                }
                if (ss + PF < s1) issue(u, ss + PF);
            }
        }
    }

    if (chunks > 1) {
        if (c != 0) red[wave][lane] = acc;
        __syncthreads();
        if (c == 0)
            for (int cc = 1; cc < chunks; ++cc) {
                const r3d_f32x4 p = red[wave + cc][lane];
                for (int i = 0; i < 4; ++i) acc[i] = acc[i] + p[i];
            }
    }
    if (c == 0 && li < M && li < MT) {
        uint16_t* yrow = Y + (int64_t)li * y_pitch;
        for (int i = 0; i < 4; ++i) {
            const int64_t n = n0 + 4 * q + i;
            if (n < N) yrow[n] = r3d_bf16_rne(acc[i]);
        }
    }
}

/* ---------------------------------------------------------------- prefill tile -----
 * 128 x 128 output tile per 256-thread workgroup (2 x 2 waves of 64 x 64), one 128-wide
 * K step per iteration staged through LDS.  Each step's MFMA results are scaled by
 * a_scale and added to f32 accumulators (the per-group flush), so the activation scale
 * is honoured exactly as in the decode kernel.  Rows past M / N stage zeros and are never
 * stored. */
constexpr int kTileM = 128, kTileN = 128;
constexpr int kWBytes = 64;                   /* mxfp4 bytes of one weight row per step */

template <int ENC>
__global__ __launch_bounds__(256) void tile_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ AS,
    const uint8_t* __restrict__ B, const void* __restrict__ BSv,
    uint16_t* __restrict__ Y,
    int M, int N, int steps, int rblk,
    int64_t a_pitch, int64_t as_pitch, int64_t b_pitch, int64_t bs_pitch, int64_t y_pitch) {
    constexpr int WB = ENC == ENC_MXFP4A8 ? 64 : 128;        /* weight bytes per row-step */
    constexpr int WP = WB + 16;                              /* padded LDS pitch */
    constexpr int AP = 128 + 16;
    __shared__ __attribute__((aligned(16))) uint8_t Ws[kTileN * WP];
    __shared__ __attribute__((aligned(16))) uint8_t As[kTileM * AP];
    __shared__ int Ss[kTileN];                               /* mxfp4: 4 E8M0 bytes per row */
    __shared__ float SAs[kTileM];
    __shared__ float SBs[kTileN];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wn = wave & 1, wm = wave >> 1;
    const int q = lane >> 4, li = lane & 15;
    const int64_t n0 = (int64_t)blockIdx.x * kTileN;
    const int64_t m0 = (int64_t)blockIdx.y * kTileM;

    r3d_f32x4 acc[4][4];
    for (int a = 0; a < 4; ++a)
        for (int b = 0; b < 4; ++b) acc[a][b] = r3d_f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    for (int s = 0; s < steps; ++s) {
        /* stage weights: kTileN rows x WB bytes, 16 bytes per thread-iteration */
        for (int idx = tid; idx < kTileN * (WB / 16); idx += 256) {
            const int r = idx / (WB / 16), cpart = idx % (WB / 16);
            const int64_t n = n0 + r;
            r3d_i32x4 v = {0, 0, 0, 0};
            if (n < N) v = r3d_ld16(B + n * b_pitch + (int64_t)s * WB + 16 * cpart);
            *reinterpret_cast<r3d_i32x4*>(Ws + r * WP + 16 * cpart) = v;
        }
        for (int idx = tid; idx < kTileM * 8; idx += 256) {
            const int r = idx >> 3, cpart = idx & 7;
            const int64_t m = m0 + r;
            r3d_i32x4 v = {0, 0, 0, 0};
            if (m < M) v = r3d_ld16(A + m * a_pitch + (int64_t)s * 128 + 16 * cpart);
            *reinterpret_cast<r3d_i32x4*>(As + r * AP + 16 * cpart) = v;
        }
        if (tid < kTileN) {
            const int64_t n = n0 + tid;
            const int64_t nc = n < N ? n : N - 1;
            if (ENC == ENC_MXFP4A8) {
                const uint8_t* bs = reinterpret_cast<const uint8_t*>(BSv) + nc * bs_pitch + 4 * (int64_t)s;
                Ss[tid] = (int)bs[0] | ((int)bs[1] << 8) | ((int)bs[2] << 16) | ((int)bs[3] << 24);
            } else {
                const uint16_t* bs = reinterpret_cast<const uint16_t*>(BSv);
                SBs[tid] = r3d_bf16_to_f32(bs[(nc / rblk) * bs_pitch + s]);
            }
        } else {
            const int r = tid - kTileN;
            const int64_t m = m0 + r;
            SAs[r] = m < M ? AS[m * as_pitch + s] : 0.0f;
        }
        __syncthreads();

        r3d_i32x8 bop[4];
        float sam[4];
        for (int mi = 0; mi < 4; ++mi) {
            const int r = wm * 64 + mi * 16 + li;
            const uint8_t* p = As + r * AP;
            const r3d_i32x4 lo = *reinterpret_cast<const r3d_i32x4*>(p + 16 * q);
            const r3d_i32x4 hi = *reinterpret_cast<const r3d_i32x4*>(p + 64 + 16 * q);
            bop[mi] = r3d_i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            sam[mi] = SAs[r];
        }
        for (int ni = 0; ni < 4; ++ni) {
            const int r = wn * 64 + ni * 16 + li;
            if (ENC == ENC_MXFP4A8) {
                const r3d_i32x4 w = *reinterpret_cast<const r3d_i32x4*>(Ws + r * WP + 16 * q);
                const int scb = (Ss[r] >> (8 * q)) & 0xFF;
                for (int mi = 0; mi < 4; ++mi) {
                    const r3d_f32x4 d = r3d_mfma_fp4_fp8(w, scb, bop[mi], R3D_E8M0_ONE);
                    for (int i = 0; i < 4; ++i) acc[ni][mi][i] = acc[ni][mi][i] + d[i] * sam[mi];
                }
            } else {
                const uint8_t* p = Ws + r * WP;
                const r3d_i32x4 lo = *reinterpret_cast<const r3d_i32x4*>(p + 16 * q);
                const r3d_i32x4 hi = *reinterpret_cast<const r3d_i32x4*>(p + 64 + 16 * q);
                const r3d_i32x8 w = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                float sbr[4];
                for (int i = 0; i < 4; ++i) sbr[i] = SBs[wn * 64 + ni * 16 + 4 * q + i];
                for (int mi = 0; mi < 4; ++mi) {
                    const r3d_f32x4 d = r3d_mfma_fp8_fp8(w, bop[mi]);
                    for (int i = 0; i < 4; ++i)
                        acc[ni][mi][i] = acc[ni][mi][i] + (d[i] * sam[mi]) * sbr[i];
                }
            }
        }
        __syncthreads();
    }

    for (int ni = 0; ni < 4; ++ni)
        for (int mi = 0; mi < 4; ++mi) {
            const int64_t m = m0 + wm * 64 + mi * 16 + li;
            if (m >= M) continue;
            uint16_t* yrow = Y + m * y_pitch;
            for (int i = 0; i < 4; ++i) {
                const int64_t n = n0 + wn * 64 + ni * 16 + 4 * q + i;
                if (n < N) yrow[n] = r3d_bf16_rne(acc[ni][mi][i]);
            }
        }
}

}  // namespace r3d

#endif /* R3D_GEMM_KERNELS_H */
