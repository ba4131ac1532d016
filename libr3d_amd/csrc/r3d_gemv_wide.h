/* r3d_gemv_wide.h -- gfx950 GEMV with K split across workgroups over launch scratch
 * (gemm_nt_q at mxfp4a8 and fp8a8, up to 64 activation rows): the tile rows' skinny band
 * and the decode rows' launches past the quad GEMV on large planes.
 *
 * The skinny band streams weights like a decode GEMV and reads each weight byte against up
 * to 64 activation rows.  A workgroup of 8 waves owns 256 weight rows (a wave TW = 2 tiles
 * of 16) and one K chunk of cg 128-wide groups; its f32 partial tile goes to plane c of
 * `part` ([kc][M][N], the launch scratch) and a second kernel sums the planes in order
 * (splitk_reduce_kernel, r3d_prefill.h).
 *
 *   * the chunk's activation rows (16 ntg of them, rows past M repeating row M - 1) and their
 *     a_scales are staged in LDS once, by direct global->LDS loads shared out over the waves:
 *     [cg groups][16 ntg rows][128 bytes], each row's eight 16-byte chunks XOR-swizzled by
 *     row % 8 (a load covers 8 whole 128-byte rows; 8 lanes reading one chunk of 8
 *     consecutive rows hit 8 distinct bank groups), then [cg][64] f32 a_scales;
 *   * each wave stages its own rows' weight scales (mxfp4a8: [RW rows][cg] E8M0 dwords;
 *     fp8a8: [cg][RW] 4-byte slots, bf16 in the low half) after them;
 *   * the weights stream in whole 128-byte lines straight into the MFMA operand registers,
 *     D lines ahead in a register ring, exactly as the line GEMV's (r3d_gemv_lines.h: two
 *     loads per 16 rows, rows 0-7 and 8-15, rebuilt by one select and two DPP rotates);
 *   * per K group, one v_mfma_scale_f32_16x16x128_f8f6f4 per (weight tile, 16-row group of
 *     activations): the weights are source A, the activation rows source B (from LDS), the
 *     E8M0 weight scales ride the scale operand (mxfp4a8); the result is scaled by the
 *     activation row's a_scale (fp8a8: then by the weight row's scale) and added to the f32
 *     accumulator -- libref's per-group flush (src/r3d_gemm_mxfp4.hip:14-15,
 *     src/r3d_gemm_fp8a8.hip:9-15).  NTG, the number of 16-row activation groups (the first
 *     ceil(M / 16)), is a template parameter, so every operand read of a K group is issued
 *     ahead of its MFMAs.
 *
 * Every load is in bounds: weight rows past N read zeros (the resource ends at the plane's
 * last row; those rows are never stored), activation rows past M repeat row M - 1, groups
 * past the chunk clamp to its last group and are never accumulated, lines past the chunk
 * are issued at offsets past the resource (answered with zeros, no memory access). */
#ifndef R3D_GEMV_WIDE_H
#define R3D_GEMV_WIDE_H

#include "r3d_device.h"
#include "r3d_gemv_lines.h"
#include "r3d_gemv_quad.h"
#include "r3d_plan.h"

namespace r3d {

template <int TW>
struct WideUnit {
    r3d_i32x4 w0[TW], w1[TW];
};

/* The small parameters packed into one argument: M (1..64) in bits 0-6, fp8a8 weight
 * scales on the 128 x 128 block grid in bit 7, activation rows at a pitch of K bytes in
 * bit 8, a_scale rows at a pitch of K / 128 floats in bit 9; and cg (< 2^16) | kc << 16 in
 * another. */
constexpr int wide_pack(int M, bool rblk128, bool a_dense, bool as_dense) {
    return M | ((int)rblk128 << 7) | ((int)a_dense << 8) | ((int)as_dense << 9);
}

/* The arguments the prologue needs come first: the hardware preloads the leading 14 dwords
 * of the argument block at dispatch (the build asks for kernel-argument preloading).  The
 * activation pitches follow them and are fetched only when the rows are not dense; part is
 * first used after the K walk.  Pitches in bytes (b, a), bf16 / E8M0 elements (bs) or
 * floats (as), all below 2^31. */
template <int ENC, int TW, int D, int NTG>
__global__ __launch_bounds__(512) void gemv_wide_kernel(
    const uint8_t* A, const float* AS, const uint8_t* B, const void* BSv,
    int N, int K, int b_pitch, int bs_pitch, int pk, int cgkc,
    int a_pitch, int as_pitch, float* __restrict__ part) {
    constexpr int ntg = NTG;                               /* 16-row activation groups */
    constexpr int G = ENC == ENC_MXFP4A8 ? 2 : 1;          /* K groups per 128-byte line */
    constexpr int WV = 8;                                  /* waves per workgroup */
    constexpr int RW = 16 * TW;                            /* weight rows per wave */
    constexpr int LPU = 2 * TW;                            /* loads per line of the ring */
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

    const int M = pk & 127;
    const bool rblk128 = (pk >> 7) & 1, a_dense = (pk >> 8) & 1, as_dense = (pk >> 9) & 1;
    const int cg = cgkc & 0xFFFF, kc = (int)((unsigned)cgkc >> 16);
    const int ntiles = (N + WV * RW - 1) / (WV * RW);      /* WV * RW = 256: a shift */
    const int sclds = ((16 * TW * cg * 4 + 255) >> 8) << 8;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

    /* unit u = chunk u / ntiles of tile u % ntiles; each XCD takes a contiguous run of units
     * (workgroups go round-robin over the 8 XCDs), so an XCD's workgroups share a chunk's
     * activation rows in its L2 */
    const int bid = blockIdx.x;
    const int units = ntiles * kc;
    const int per = units >> 3, rem = units & 7, x = bid & 7;
    const int u = x * per + (x < rem ? x : rem) + (bid >> 3);
    const int c = u / ntiles, t = u - c * ntiles;
    const int groups = K >> 7;
    const int g0 = c * cg;                                 /* a multiple of G */
    const int gc = groups - g0 < cg ? groups - g0 : cg;    /* >= 1: no empty chunk */
    const int lines = (gc + G - 1) / G;
    const int u0 = g0 / G;                                 /* first line of the chunk */
    const int64_t n0 = (int64_t)t * (WV * RW) + wave * RW;

    const int p = lane & 15;            /* row of src A / column of src B inside a tile */
    const bool first = p < 8;
    const int kb = lane >> 4;
    const int r8 = lane & 7;

    /* ---- 1. LDS staging, issued before the weight ring so the ring's waits cover it */
    const int rows8 = 2 * ntg;                             /* 8-row images per group */
    const int gstride = ntg * 2048;                        /* bytes of one group's rows */
    const int xs_off = cg * gstride;
    const int sc_off = xs_off + cg * 256;
    const uint32_t sbase = (uint32_t)(uintptr_t)smem;
    {
        const int tm = (lane >> 3) & 7;                    /* row of this lane in an image */
        const int ch = (lane & 7) ^ tm;                    /* the chunk it fetches */
        /* dense rows take their pitch from K, so a_pitch / as_pitch (arguments past the
         * preloaded ones) are fetched on the other branches only */
        auto stage_x = [&](int64_t ap) {
            for (int i = wave; i < gc * rows8; i += WV) {
                const int gi = i / rows8, ri = i - gi * rows8;
                int m = 8 * ri + tm;
                if (m > M - 1) m = M - 1;
                r3d_quad_dma<16>(A + (int64_t)m * ap + 128 * (int64_t)(g0 + gi) + 16 * ch,
                                 sbase + (uint32_t)(gi * gstride + ri * 1024));
            }
        };
        if (a_dense) stage_x(K);
        else stage_x(a_pitch);
        auto stage_as = [&](int64_t asp) {
            for (int gi = wave; gi < gc; gi += WV) {
                const int m = lane < M ? lane : M - 1;
                r3d_quad_dma<4>(AS + (int64_t)m * asp + g0 + gi,
                                sbase + (uint32_t)(xs_off + 256 * gi));
            }
        };
        if (as_dense) stage_as(groups);
        else stage_as(as_pitch);
    }
    const uint32_t wl = sbase + (uint32_t)(sc_off + wave * sclds);
    if (ENC == ENC_MXFP4A8) {
        /* [RW rows][cg] E8M0 dwords */
        const uint8_t* BS8 = reinterpret_cast<const uint8_t*>(BSv);
        for (int h = 0; h < (sclds >> 8); ++h) {
            const int e = lane + 64 * h;
            int r = e / cg, d = e - r * cg;
            if (r > RW - 1) { r = RW - 1; d = cg - 1; }
            if (d > gc - 1) d = gc - 1;
            const int64_t nr = n0 + r < N ? n0 + r : N - 1;
            r3d_quad_dma<4>(BS8 + nr * bs_pitch + 4 * (int64_t)(g0 + d), wl + 256 * h);
        }
    } else {
        /* [cg][RW rows] 4-byte slots, bf16 in the low half */
        const uint16_t* BS16 = reinterpret_cast<const uint16_t*>(BSv);
        for (int h = 0; h < (sclds >> 8); ++h) {
            const int e = lane + 64 * h;
            int d = e / RW;
            const int r = e % RW;
            if (d > gc - 1) d = gc - 1;
            const int64_t nr = n0 + r < N ? n0 + r : N - 1;
            const int64_t sr = rblk128 ? nr >> 7 : nr;
            r3d_quad_dma<2>(BS16 + sr * bs_pitch + g0 + d, wl + 256 * h);
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    /* ---- 2. the weight stream over the wave's rows and the chunk's lines.  The resource ends
     * where the plane's rows end, so rows past N (and a line running past K: mxfp4a8 with an
     * odd group count) read zeros. */
    const int64_t rows = N - n0 < RW ? (N - n0 > 0 ? N - n0 : 0) : RW;   /* 0: an empty wave */
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(B + n0 * b_pitch), (short)0, (int)(rows * b_pitch), 0x00020000);
    const int ca = p < 8 ? kb : 4 + kb, cb = p < 8 ? 4 + kb : kb;
    uint32_t wa[TW], wb[TW];
#pragma unroll
    for (int tt = 0; tt < TW; ++tt) {
        wa[tt] = (uint32_t)((16 * tt + r8) * b_pitch + 16 * ca + 128 * (int64_t)u0);
        wb[tt] = (uint32_t)((16 * tt + 8 + r8) * b_pitch + 16 * cb + 128 * (int64_t)u0);
    }
    using Unit = WideUnit<TW>;
    const uint32_t kSkip = 0x80000000u;
    /* the selected offsets are pinned in registers (see r3d_gemv_lines.h): the compiler
     * would otherwise branch around the skipped form with a full wait */
    auto off = [](bool in, uint32_t o, uint32_t skip) {
        uint32_t v = in ? o : skip;
        asm volatile("" : "+v"(v));
        return v;
    };
    auto load = [&](int s) {
        const bool in = s < lines;
        Unit v;
#pragma unroll
        for (int tt = 0; tt < TW; ++tt) {
            v.w0[tt] = r3d_buf_ld16_stream(wrs, off(in, wa[tt] + 128u * (uint32_t)s, kSkip + 128 * tt));
            v.w1[tt] = r3d_buf_ld16_stream(wrs, off(in, wb[tt] + 128u * (uint32_t)s,
                                                    kSkip + 128 * tt + 64));
        }
        return v;
    };
    Unit ring[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        ring[d] = load(d);
        __builtin_amdgcn_sched_barrier(0);
    }
    /* the staging loads are all but the newest D * LPU loads in flight: wait for them, then
     * meet the other waves (the activation rows are shared) */
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" :: "n"(D * LPU) : "memory");

    /* ---- 3. consume: B operand and a_scales of activation group tg from LDS */
    const int xlo = 16 * (kb ^ (p & 7)), xhi = 16 * ((kb + 4) ^ (p & 7));
    const float* xs = reinterpret_cast<const float*>(smem + xs_off);
    const uint8_t* sc = smem + sc_off + wave * sclds;
    r3d_f32x4 acc[TW][NTG];
#pragma unroll
    for (int tt = 0; tt < TW; ++tt)
#pragma unroll
        for (int g = 0; g < NTG; ++g) acc[tt][g] = r3d_f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    auto consume = [&](const Unit& v, int s) {
        r3d_i32x4 wlo[TW], whi[TW];
#pragma unroll
        for (int tt = 0; tt < TW; ++tt) r3d_lines_fix(v.w0[tt], v.w1[tt], first, wlo[tt], whi[tt]);
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const int gl = G * s + h;                      /* group inside the chunk */
            const bool live = gl < gc;
            const int gr = live ? gl : gc - 1;
            const uint8_t* xg = smem + gr * gstride + 128 * p;
            /* every activation group's operand and a_scale first, then the MFMAs */
            r3d_i32x8 bvs[NTG];
            float ass[NTG];
#pragma unroll
            for (int tg = 0; tg < NTG; ++tg) {
                const r3d_i32x4 lo = *reinterpret_cast<const r3d_i32x4*>(xg + 2048 * tg + xlo);
                const r3d_i32x4 hi = *reinterpret_cast<const r3d_i32x4*>(xg + 2048 * tg + xhi);
                bvs[tg] = r3d_i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                ass[tg] = xs[gr * 64 + 16 * tg + p];
            }
#pragma unroll
            for (int tg = 0; tg < NTG; ++tg) {
                const r3d_i32x8 bv = bvs[tg];
                const float a_s = ass[tg];
#pragma unroll
                for (int tt = 0; tt < TW; ++tt) {
                    if (ENC == ENC_MXFP4A8) {
                        const int sa = sc[(16 * tt + p) * 4 * cg + 4 * gr + kb];   /* row, block kb */
                        const r3d_f32x4 dv =
                            r3d_mfma_fp4_fp8(h == 0 ? wlo[tt] : whi[tt], sa, bv, R3D_E8M0_ONE);
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[tt][tg][i] += live ? dv[i] * a_s : 0.0f;
                    } else {
                        const r3d_i32x8 av = {wlo[tt][0], wlo[tt][1], wlo[tt][2], wlo[tt][3],
                                              whi[tt][0], whi[tt][1], whi[tt][2], whi[tt][3]};
                        const r3d_f32x4 dv = r3d_mfma_fp8_fp8(av, bv);
                        /* the result rows of this lane are 4 kb .. 4 kb + 3 of tile tt */
                        const r3d_i32x4 sb = *reinterpret_cast<const r3d_i32x4*>(
                            sc + 4 * (gr * RW + 16 * tt + 4 * kb));
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const float sbv = __uint_as_float((uint32_t)sb[i] << 16);
                            acc[tt][tg][i] += live ? (dv[i] * a_s) * sbv : 0.0f;
                        }
                    }
                }
            }
        }
    };

    int s0 = 0;
    for (; s0 + 2 * D <= lines; s0 += D) {
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
        if (s0 + D + d < lines) consume(ring[d], s0 + D + d);
        __builtin_amdgcn_sched_barrier(0);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   /* the skipped loads past the chunk */
    /* every accumulator is complete here, in every lane: the compiler may otherwise sink the
     * last line's MFMAs (and the per-lane operand selects feeding them) into the stores'
     * lane-divergent branches, where lanes off the exec mask would hand the MFMA stale
     * operands */
#pragma unroll
    for (int tt = 0; tt < TW; ++tt)
#pragma unroll
        for (int tg = 0; tg < NTG; ++tg) asm volatile("" : "+v"(acc[tt][tg]));

    /* ---- 4. the partial tile: lane l holds rows 4 (l / 16) + i of each weight tile for
     * activation row 16 tg + l % 16 -- four consecutive columns of plane c */
    float* pp = part + (int64_t)c * M * N;
    const bool v4 = (N & 3) == 0;
#pragma unroll
    for (int tt = 0; tt < TW; ++tt)
#pragma unroll
        for (int tg = 0; tg < NTG; ++tg) {
            const int m = 16 * tg + p;
            const int64_t n = n0 + 16 * tt + 4 * kb;
            if (m >= M || n >= N) continue;
            float* d = pp + (int64_t)m * N + n;
            const r3d_f32x4 v = acc[tt][tg];
            if (v4) {
                *reinterpret_cast<r3d_f32x4*>(d) = v;
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (n + i < N) d[i] = v[i];
            }
        }
}

}  // namespace r3d

#endif /* R3D_GEMV_WIDE_H */
