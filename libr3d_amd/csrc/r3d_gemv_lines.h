/* r3d_gemv_lines.h -- gfx950 decode GEMV for 5..16 activation rows (gemm_nt_q at mxfp4a8
 * and fp8a8).  (MT = 8 also serves M <= 4 correctly; the launch policy sends those to the
 * quad GEMV or the 16-row GEMV, measured faster there.)
 *
 * One wave owns a 16-row weight tile and one contiguous chunk of K; v_mfma_scale_f32_16x
 * 16x128_f8f6f4 takes the 16 weight rows as source A and 16 activation rows as source B,
 * so every product of the MFMA is used.  The unit of the walk is a LINE: 128 contiguous
 * bytes of every weight row -- one 128-wide K group at fp8a8, two at mxfp4a8 (64 bytes of
 * e2m1 codes per group).  A wave fetches a unit with two buffer_load_dwordx4, the first
 * covering rows 0-7 and the second rows 8-15, each in whole 128-byte lines (an
 * instruction walking all 16 rows could only cover half lines, which streams ~25 % slower
 * on MI355X).  The activation rows of each group arrive the same way (rows 0-7, rows
 * 8-15) straight into registers, from L2: at M = 16 they are as many bytes per group as
 * the weights, far too many to stage whole in LDS, and every wave reads them in the same
 * order as its weights.
 *
 * Register shuffle.  Inside one 16-lane row of the wave, the first load gives lane p the
 * 16-byte chunk ca = kb (p < 8) or 4 + kb (p >= 8) of row p % 8, and the second load the
 * chunk cb = 4 + kb (p < 8) or kb (p >= 8) of row 8 + p % 8 (kb = lane / 16).  Then
 *     lo = (p < 8 ? load0 : load1)            -> row p, chunk kb
 *     hi = row_ror:8 of (p < 8 ? load1 : load0) -> row p, chunk 4 + kb
 * (one select and two DPP rotates per register).  For an fp8 operand (lo,
 * hi) are exactly the MFMA's bytes [16kb, +16) and [64 + 16kb, +16) of the lane's row;
 * for e2m1 weights lo is the lane's 32-wide block of the line's first group and hi that of
 * the second.  The per-group sums are then libref's per-group subs: the a_scale (and the
 * fp8a8 weight scale) multiply the MFMA result per group (src/r3d_gemm_mxfp4.hip:14-15,
 * src/r3d_gemm_fp8a8.hip:9-15), the E8M0 weight scales ride the MFMA's scale operand.
 *
 * The ring, the skipped loads past a chunk (offsets >= 2^31 that the buffer range check
 * answers with zeros) and the inline-asm LDS staging follow the quad GEMV
 * (r3d_gemv_quad.h): each wave stages its own activation scales ([16][gmax] f32) and
 * weight scales (mxfp4a8: [16 rows][gmax] E8M0 dwords; fp8a8: [gmax][16 rows] 4-byte
 * slots, bf16 in the low half) in its wlds-byte slice of LDS, then primes the ring.
 *
 * Work split: a workgroup is 4 waves = (4 / chunks) tiles x chunks; the chunks of a tile
 * fold through LDS in a fixed order (deterministic).  Rows past N clamp to row N-1,
 * activation rows past M duplicate row M-1, groups past a chunk clamp to its last group;
 * none of these is accumulated or stored. */
#ifndef R3D_GEMV_LINES_H
#define R3D_GEMV_LINES_H

#include "r3d_device.h"
#include "r3d_gemv_quad.h"
#include "r3d_plan.h"

namespace r3d {

/* (lo, hi) operand registers from the two loads of a line pair (see the header); `first`
 * is true in lanes 0-7 of every 16-lane row. */
__device__ __forceinline__ void r3d_lines_fix(const r3d_i32x4& a, const r3d_i32x4& b, bool first,
                                              r3d_i32x4& lo, r3d_i32x4& hi) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        lo[i] = first ? a[i] : b[i];
        /* every lane takes b from lane p ^ 8, then lanes 0-7 (banks 0-1) take a from it */
        const int t = __builtin_amdgcn_mov_dpp(b[i], 0x128, 0xF, 0xF, false);   /* row_ror:8 */
        hi[i] = __builtin_amdgcn_update_dpp(t, a[i], 0x128, 0xF, 0x3, false);
    }
}

/* One unit of one wave in the ring: the line pairs of its TW weight tiles and, per group of
 * the unit, the activation pair (only the rows 0-7 load when MT is 8). */
template <int ENC, int MT, int TW>
struct LinesUnit {
    static constexpr int G = ENC == ENC_MXFP4A8 ? 2 : 1;
    r3d_i32x4 w0[TW], w1[TW];
    r3d_i32x4 x0[G];
    r3d_i32x4 x1[MT == 16 ? G : 1];
};

/* The small parameters packed into one argument: M (1..64: the skinny band's passes see
 * up to 16 each) in bits 0-6, log2 of the chunk count (0..2) in bits 7-8, fp8a8 weight
 * scales on the 128 x 128 block grid in bit 9, a_scale rows at a pitch of K / 128 floats
 * in bit 10. */
constexpr int lines_pack(int M, int log2_chunks, bool rblk128, bool as_dense) {
    return M | (log2_chunks << 7) | ((int)rblk128 << 9) | ((int)as_dense << 10);
}

/* The arguments the prologue needs come first (the hardware preloads the leading 14 dwords
 * of the argument block at dispatch); as_pitch (rows not dense), Y and its pitch follow.
 * Pitches in bytes (b, a), bf16 / E8M0 elements (bs) or floats (as), below 2^31. */
template <int ENC, int MT, int TW, int D>
__global__ __launch_bounds__(256) void gemv_lines_kernel(
    const uint8_t* A, const float* AS, const uint8_t* B, const void* BSv,
    int N, int K, int b_pitch, int bs_pitch, int a_pitch, int pk,
    int as_pitch, uint16_t* __restrict__ Y, int64_t y_pitch) {
    constexpr int G = ENC == ENC_MXFP4A8 ? 2 : 1;          /* K groups per unit */
    constexpr int LPU = 2 * TW + G * (MT == 16 ? 2 : 1);   /* loads per unit */
    constexpr int RW = 16 * TW;                            /* weight rows per wave */
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    int M = pk & 127;
    const int cl = (pk >> 7) & 3, chunks = 1 << cl;
    const bool rblk128 = (pk >> 9) & 1, as_dense = (pk >> 10) & 1;
    const int groups = K >> 7;
    /* grid.y > 1 (the skinny band): workgroup row y computes activation rows
     * [16 y, 16 y + 16) of a taller A -- the same arithmetic as a 16-row call (AS moves
     * with it in the staging below) */
    const int m0 = 16 * (int)blockIdx.y;
    {
        A += (int64_t)m0 * a_pitch;
        Y += m0 * y_pitch;
        M = M - m0 < 16 ? M - m0 : 16;
    }

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int units = (groups + G - 1) / G;
    const int tpb = 4 >> cl;                               /* row blocks per workgroup */
    const int ti = wave >> cl, c = wave & (chunks - 1);
    const int64_t n0 = ((int64_t)blockIdx.x * tpb + ti) * RW;
    const int u0 = (units * c) >> cl;                      /* units < 2^21: no overflow */
    const int ns = ((units * (c + 1)) >> cl) - u0;         /* >= 1: chunks <= units */
    const int gmax = G * ((units + chunks - 1) >> cl);
    const int wlds = lines_wlds(ENC, TW, K, chunks);
    __builtin_assume(ns >= 1);
    const int g0 = G * u0;
    const int gc = (G * ns < groups - g0) ? G * ns : groups - g0;   /* real groups */

    const int p = lane & 15;           /* row of src A / column of src B inside a tile */
    const bool first = p < 8;
    const int kb = lane >> 4;
    const int r8 = lane & 7;

    /* ---- 1. LDS staging of this wave's scales: a_scales [16][gmax] f32 in the first xsb
     * bytes of its slice, then the weight scales of its RW rows */
    const int xsb = (64 * gmax + 255) & ~255;
    const uint32_t wl = (uint32_t)(uintptr_t)smem + (uint32_t)(wave * wlds);
    /* dense a_scale rows take their pitch from K, so as_pitch (an argument past the
     * preloaded ones) is fetched on the other branch only */
    auto stage_as = [&](int64_t asp) {
        for (int h = 0; h < (xsb >> 8); ++h) {
            const int e = lane + 64 * h;
            int t = e / gmax, g = e - t * gmax;
            if (t > 15) { t = 15; g = gmax - 1; }
            if (g > gc - 1) g = gc - 1;
            const int tm = t < M ? t : M - 1;
            r3d_quad_dma<4>(AS + (int64_t)(m0 + tm) * asp + g0 + g, wl + 256 * h);
        }
    };
    if (as_dense) stage_as(groups);
    else stage_as(as_pitch);
    const int nsc = (wlds - xsb) >> 8;
    if (ENC == ENC_MXFP4A8) {
        /* [RW rows][gmax] E8M0 dwords */
        const uint8_t* BS8 = reinterpret_cast<const uint8_t*>(BSv);
        for (int h = 0; h < nsc; ++h) {
            const int e = lane + 64 * h;
            int r = e / gmax, d = e - r * gmax;
            if (r > RW - 1) { r = RW - 1; d = gmax - 1; }
            if (d > gc - 1) d = gc - 1;
            const int64_t nr = n0 + r < N ? n0 + r : N - 1;
            r3d_quad_dma<4>(BS8 + nr * bs_pitch + 4 * (int64_t)(g0 + d), wl + xsb + 256 * h);
        }
    } else {
        /* [gmax][RW rows] 4-byte slots, bf16 in the low half */
        const uint16_t* BS16 = reinterpret_cast<const uint16_t*>(BSv);
        for (int h = 0; h < nsc; ++h) {
            const int e = lane + 64 * h;
            int d = e / RW;
            const int r = e % RW;
            if (d > gc - 1) d = gc - 1;
            const int64_t nr = n0 + r < N ? n0 + r : N - 1;
            const int64_t sr = rblk128 ? nr >> 7 : nr;
            r3d_quad_dma<2>(BS16 + sr * bs_pitch + g0 + d, wl + xsb + 256 * h);
        }
    }

    /* ---- 2. the streams: weights over the wave's rows, activations over the A plane.  The
     * resources end where the operands end, so a line running past K (mxfp4a8 with an odd
     * group count) reads zeros, never past the plane. */
    const int64_t rows = N - n0 < RW ? (N - n0 > 0 ? N - n0 : 0) : RW;   /* 0: an empty block */
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(B + n0 * b_pitch), (short)0, (int)(rows * b_pitch), 0x00020000);
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(A), (short)0, (int)((int64_t)(M - 1) * a_pitch + K), 0x00020000);
    const int ca = p < 8 ? kb : 4 + kb, cb = p < 8 ? 4 + kb : kb;
    uint32_t wa[TW], wb[TW];
#pragma unroll
    for (int t = 0; t < TW; ++t) {
        const int64_t ra = n0 + 16 * t + r8 < N ? n0 + 16 * t + r8 : N - 1;
        const int64_t rb = n0 + 16 * t + 8 + r8 < N ? n0 + 16 * t + 8 + r8 : N - 1;
        wa[t] = (uint32_t)((ra - n0) * b_pitch + 16 * ca);
        wb[t] = (uint32_t)((rb - n0) * b_pitch + 16 * cb);
    }
    const int ta = r8 < M ? r8 : M - 1, tb = 8 + r8 < M ? 8 + r8 : M - 1;
    const uint32_t xa = (uint32_t)(ta * a_pitch + 16 * ca);
    const uint32_t xb = (uint32_t)(tb * a_pitch + 16 * cb);

    using Unit = LinesUnit<ENC, MT, TW>;
    const uint32_t kSkip = 0x80000000u;
    /* The selected offsets are pinned in registers: left alone, the compiler folds the step's
     * constant part of the real offset into the instruction's immediate, which no longer
     * matches the skipped form, and branches around the load (with a full wait).  Skipped
     * offsets differ per load so that no two loads can be merged. */
    auto off = [](bool in, uint32_t o, uint32_t skip) {
        uint32_t v = in ? o : skip;
        asm volatile("" : "+v"(v));
        return (int)v;
    };
    auto load = [&](int s) {
        const bool in = s < ns;
        const uint32_t u = (uint32_t)(u0 + s);
        Unit v;
#pragma unroll
        for (int t = 0; t < TW; ++t) {
            v.w0[t] = r3d_buf_ld16_stream(wrs, (uint32_t)off(in, wa[t] + 128u * u, kSkip + 128 * t));
            v.w1[t] = r3d_buf_ld16_stream(wrs, (uint32_t)off(in, wb[t] + 128u * u, kSkip + 128 * t + 64));
        }
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const int gg = G * (u0 + s) + h;
            const uint32_t g = (uint32_t)(gg < groups ? gg : groups - 1);
            v.x0[h] = __builtin_bit_cast(r3d_i32x4, __builtin_amdgcn_raw_buffer_load_b128(
                xrs, off(in, xa + 128u * g, kSkip + 1024 + 256 * h), 0, 0));
            if (MT == 16)
                v.x1[h] = __builtin_bit_cast(r3d_i32x4, __builtin_amdgcn_raw_buffer_load_b128(
                    xrs, off(in, xb + 128u * g, kSkip + 1024 + 256 * h + 128), 0, 0));
        }
        return v;
    };

    Unit ring[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        ring[d] = load(d);
        __builtin_amdgcn_sched_barrier(0);
    }
    /* the staging loads are all but the newest D * LPU loads in flight */
    asm volatile("s_waitcnt vmcnt(%0)" :: "n"(D * LPU) : "memory");

    /* ---- 3. consume */
    const float* xs = reinterpret_cast<const float*>(smem + wave * wlds) + p * gmax;
    const uint8_t* sc = smem + wave * wlds + xsb;
    r3d_f32x4 acc[TW];
#pragma unroll
    for (int t = 0; t < TW; ++t) acc[t] = r3d_f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    auto consume = [&](const Unit& v, int s) {
        r3d_i32x4 wlo[TW], whi[TW];
#pragma unroll
        for (int t = 0; t < TW; ++t) r3d_lines_fix(v.w0[t], v.w1[t], first, wlo[t], whi[t]);
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const int gl = G * s + h;                      /* group inside the chunk */
            const bool live = gl < gc;
            const int gr = live ? gl : gc - 1;
            r3d_i32x4 xlo, xhi;
            if (MT == 16) {
                r3d_lines_fix(v.x0[h], v.x1[h], first, xlo, xhi);
            } else {
                /* columns 8-15 of the result are never stored: only rows p < 8 of B matter */
                xlo = v.x0[h];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    xhi[i] = __builtin_amdgcn_mov_dpp(v.x0[h][i], 0x128, 0xF, 0xF, false);
            }
            const r3d_i32x8 bv = {xlo[0], xlo[1], xlo[2], xlo[3], xhi[0], xhi[1], xhi[2], xhi[3]};
            const float a_s = xs[gr];
#pragma unroll
            for (int t = 0; t < TW; ++t) {
                if (ENC == ENC_MXFP4A8) {
                    const int sa = sc[(16 * t + p) * 4 * gmax + 4 * gr + kb];   /* row, block kb */
                    const r3d_f32x4 dv =
                        r3d_mfma_fp4_fp8(h == 0 ? wlo[t] : whi[t], sa, bv, R3D_E8M0_ONE);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[t][i] += live ? dv[i] * a_s : 0.0f;
                } else {
                    const r3d_i32x8 av = {wlo[t][0], wlo[t][1], wlo[t][2], wlo[t][3],
                                          whi[t][0], whi[t][1], whi[t][2], whi[t][3]};
                    const r3d_f32x4 dv = r3d_mfma_fp8_fp8(av, bv);
                    /* the result rows of this lane are 4 kb .. 4 kb + 3 of tile t */
                    const r3d_i32x4 sb = *reinterpret_cast<const r3d_i32x4*>(
                        sc + 4 * (gr * RW + 16 * t + 4 * kb));
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float sbv = __uint_as_float((uint32_t)sb[i] << 16);
                        acc[t][i] += live ? (dv[i] * a_s) * sbv : 0.0f;
                    }
                }
            }
        }
    };

    int s0 = 0;
    for (; s0 + 2 * D <= ns; s0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            consume(ring[d], s0 + d);
            ring[d] = load(s0 + d + D);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
        consume(ring[d], s0 + d);
        ring[d] = load(s0 + d + D);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
        if (s0 + D + d < ns) consume(ring[d], s0 + D + d);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int t = 0; t < TW; ++t) asm volatile("" : "+v"(acc[t]));   /* no MFMA sinks below */

    /* ---- 4. fold: lane l holds rows 4 (l / 16) + i of each tile for activation row l % 16 */
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");   /* LDS reads done */
    r3d_f32x4* red = reinterpret_cast<r3d_f32x4*>(smem);
#pragma unroll
    for (int t = 0; t < TW; ++t) red[(wave * TW + t) * 64 + lane] = acc[t];
    __syncthreads();
    const float* rf = reinterpret_cast<const float*>(smem);
    for (int o = threadIdx.x; o < tpb * RW * MT; o += 256) {
        const int r = o % RW, tk = (o / RW) % MT, b = o / (RW * MT);
        const int t = r >> 4, rr = r & 15;
        float y = 0.0f;
        for (int cc = 0; cc < chunks; ++cc)
            y += rf[(((b * chunks + cc) * TW + t) * 64 + 16 * (rr >> 2) + tk) * 4 + (rr & 3)];
        const int64_t n = ((int64_t)blockIdx.x * tpb + b) * RW + r;
        if (tk < M && n < N) Y[(int64_t)tk * y_pitch + n] = r3d_bf16_rne(y);
    }
}

}  // namespace r3d

#endif /* R3D_GEMV_LINES_H */
