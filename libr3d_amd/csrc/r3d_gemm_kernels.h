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
#include "r3d_gemv_layout.h"

namespace r3d {

/* ---------------------------------------------------------------- decode GEMV ------
 * One wave owns a 16-row weight tile and one contiguous chunk of its K steps; the
 * `chunks` waves of a tile sit in the same workgroup and fold their f32 partials through
 * LDS in chunk order (deterministic).
 *
 * The chunk is walked in runs of kRunBytes bytes per weight row.  Everything a run needs
 * -- the 16 weight rows, the activation rows, the weight scales and the activation
 * scales -- arrives by direct global->LDS loads (global_load_lds, 16 bytes per lane for
 * the planes, 2 or 4 for the scales), issued one run ahead into the other half of a
 * double buffer.  Each weight instruction reads 512 contiguous bytes of two rows: HBM
 * streams contiguous bursts, where the MFMA operand's native 16-rows-per-instruction walk
 * measured well under two thirds of that on MI355X.  The only wait in the steady state is
 * vmcnt(<loads of the next run>), so the next run is always in flight while this one is
 * consumed from LDS.  Odd rows store their 16-byte chunks pairwise swapped so the MFMA
 * operand reads (16 rows at one offset) spread over the LDS banks.
 *
 * Every load is unconditional and in bounds: weight rows n >= N clamp to row N-1,
 * activation rows m >= M duplicate row M-1, a short last run clamps its lanes inside the
 * chunk, and nothing clamped is ever used or stored. */
template <int ENC, int MT>
__global__ __launch_bounds__(512) void gemv_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ AS,
    const uint8_t* __restrict__ B, const void* __restrict__ BSv,
    uint16_t* __restrict__ Y,
    int M, int N, int steps, int chunks, int rblk,
    int64_t a_pitch, int64_t as_pitch, int64_t b_pitch, int64_t bs_pitch, int64_t y_pitch) {
    using L = GemvLayout<ENC, MT>;
    constexpr int SB = L::SB, RS = L::RS;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int waves = blockDim.x >> 6;
    const int tpb = waves / chunks;
    const int64_t tile = (int64_t)blockIdx.x * tpb + wave / chunks;
    const int c = wave % chunks;
    const int s0 = (int)((int64_t)steps * c / chunks);
    const int s1 = (int)((int64_t)steps * (c + 1) / chunks);

    const int q = lane >> 4;           /* K sub-block of this lane inside a step */
    const int li = lane & 15;          /* weight row (src A) / activation row (src B) */
    const int64_t n0 = tile * 16;
    uint8_t* wbase = smem + wave * L::WAVE;

    /* ---- issue side: lane roles for the direct loads (all wave-uniform LDS bases) */
    const int pr = lane >> 5;                         /* row within a weight pair */
    const int pc = (lane & 31) ^ pr;                  /* chunk this lane fetches (odd rows swap) */
    const uint16_t* BS16 = reinterpret_cast<const uint16_t*>(BSv);
    const uint8_t* BS8 = reinterpret_cast<const uint8_t*>(BSv);

    auto issue = [&](int rs, int ns, uint8_t* buf) {
        /* weights: pair p = rows 2p, 2p+1; lane -> row 2p+pr, chunk pc (clamped in run) */
        const int rl = ns * SB;
        const int wo = (16 * pc < rl - 16) ? 16 * pc : rl - 16;
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            int64_t nr = n0 + 2 * p + pr;
            if (nr > N - 1) nr = N - 1;
            r3d_lds_load(B + nr * b_pitch + (int64_t)rs * SB + wo, buf + L::W + p * kPairPitch, 16);
        }
        /* activations: token t's run bytes [128 rs, +1024) (fp8 runs use the first 512) */
        {
            const int ab = ns * 128;
            const int ao = (16 * lane < ab - 16) ? 16 * lane : ab - 16;
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const int tm = t < M ? t : M - 1;
                r3d_lds_load(A + (int64_t)tm * a_pitch + (int64_t)rs * 128 + ao, buf + L::AC + t * 1040, 16);
            }
        }
        /* weight scales */
        if (ENC == ENC_MXFP4A8) {
            /* [16 rows][RS dwords]: lane -> row (lane / RS) + 8h, dword lane % RS (clamped) */
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int row = (lane / RS) + 8 * h;
                int64_t nr = n0 + row;
                if (nr > N - 1) nr = N - 1;
                const int d = (lane % RS) < ns ? (lane % RS) : ns - 1;
                r3d_lds_load(BS8 + nr * bs_pitch + 4 * ((int64_t)rs + d), buf + L::SC + h * 256, 4);
            }
        } else {
            /* [16 rows][RS] slots of 4 bytes (bf16 in the low half): lane -> row lane / RS,
             * step lane % RS (clamped) */
            const int row = lane / RS;
            int64_t nr = n0 + row;
            if (nr > N - 1) nr = N - 1;
            const int d = (lane % RS) < ns ? (lane % RS) : ns - 1;
            r3d_lds_load(BS16 + (nr / rblk) * bs_pitch + rs + d, buf + L::SC, 2);
        }
        /* activation scales: [MT][RS] f32, 64 per instruction */
#pragma unroll
        for (int h = 0; h < L::N_AS; ++h) {
            const int e = lane + 64 * h;
            int t = e / RS;
            if (t > MT - 1) t = MT - 1;
            const int tm = t < M ? t : M - 1;
            const int d = (e % RS) < ns ? (e % RS) : ns - 1;
            r3d_lds_load(AS + (int64_t)tm * as_pitch + rs + d, buf + L::AS + h * 256, 4);
        }
    };

    /* ---- consume side */
    const int wrow_off = L::W + (li >> 1) * kPairPitch + (li & 1) * kRunBytes;
    const int wsw = li & 1;
    const int tok = MT == 1 ? 0 : li;
    r3d_f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};

    auto consume = [&](const uint8_t* buf, int j) {
        const uint8_t* ap = buf + L::AC + tok * 1040 + 128 * j + 16 * q;
        const r3d_i32x4 alo = *reinterpret_cast<const r3d_i32x4*>(ap);
        const r3d_i32x4 ahi = *reinterpret_cast<const r3d_i32x4*>(ap + 64);
        const r3d_i32x8 av = {alo[0], alo[1], alo[2], alo[3], ahi[0], ahi[1], ahi[2], ahi[3]};
        const float a_s = *reinterpret_cast<const float*>(buf + L::AS + 4 * (tok * RS + j));
        if (ENC == ENC_MXFP4A8) {
            const int ch = (4 * j + q) ^ wsw;
            const r3d_i32x4 w = *reinterpret_cast<const r3d_i32x4*>(buf + wrow_off + 16 * ch);
            const int sc = buf[L::SC + li * 4 * RS + 4 * j + q];
            const r3d_f32x4 d = r3d_mfma_fp4_fp8(w, sc, av, R3D_E8M0_ONE);
            for (int i = 0; i < 4; ++i) acc[i] = acc[i] + d[i] * a_s;
        } else {
            const int c0 = (8 * j + q) ^ wsw, c1 = (8 * j + 4 + q) ^ wsw;
            const r3d_i32x4 lo = *reinterpret_cast<const r3d_i32x4*>(buf + wrow_off + 16 * c0);
            const r3d_i32x4 hi = *reinterpret_cast<const r3d_i32x4*>(buf + wrow_off + 16 * c1);
            const r3d_i32x8 w = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            const r3d_f32x4 d = r3d_mfma_fp8_fp8(w, av);
            /* a 2-byte direct load still fills one 4-byte LDS slot per lane */
            const uint32_t* sbp = reinterpret_cast<const uint32_t*>(buf + L::SC);
            for (int i = 0; i < 4; ++i) {
                const float sbv = __uint_as_float(sbp[(4 * q + i) * RS + j] << 16);
                acc[i] = acc[i] + (d[i] * a_s) * sbv;
            }
        }
    };

    /* ---- walk: with two buffers, run r+1 is in flight while run r is consumed */
    const int nrun = (s1 - s0 + RS - 1) / RS;
    if (L::DB == 2 && nrun > 0) issue(s0, (s1 - s0) < RS ? (s1 - s0) : RS, wbase);
    for (int r = 0; r < nrun; ++r) {
        uint8_t* cur = wbase + (L::DB == 2 ? (r & 1) * L::BUF : 0);
        const int rs = s0 + r * RS;
        const int ns = (s1 - rs) < RS ? (s1 - rs) : RS;
        if (L::DB == 1) {
            issue(rs, ns, cur);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        } else if (r + 1 < nrun) {
            const int rn = rs + RS;
            issue(rn, (s1 - rn) < RS ? (s1 - rn) : RS, wbase + ((r + 1) & 1) * L::BUF);
            asm volatile("s_waitcnt vmcnt(%0)" :: "n"(L::LOADS) : "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        if (ns == RS) {
#pragma unroll
            for (int j = 0; j < RS; ++j) consume(cur, j);
        } else {
            for (int j = 0; j < ns; ++j) consume(cur, j);
        }
        /* this buffer is refilled by a later issue: its reads are done */
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }

    if (chunks > 1) {
        __syncthreads();                                  /* every wave is done with LDS */
        r3d_f32x4* red = reinterpret_cast<r3d_f32x4*>(smem);
        if (c != 0) red[wave * 64 + lane] = acc;
        __syncthreads();
        if (c == 0)
            for (int cc = 1; cc < chunks; ++cc) {
                const r3d_f32x4 p = red[(wave + cc) * 64 + lane];
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
