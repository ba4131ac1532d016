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

}  // namespace r3d

#endif /* R3D_GEMM_KERNELS_H */
