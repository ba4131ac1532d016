/* r3d_prefill.h -- the prefill GEMM of the mxfp4 gemm_nt_q rows on CDNA4 block-scaled
 * MFMA, and the bf16 -> mxfp8 activation quantiser that feeds its bf16-in row.
 *
 * Y[m, n] = sum_k A[m, k] * W[n, k], W in mxfp4 (e2m1 codes + one E8M0 per 32 along K),
 * A in e4m3.  A workgroup of 4 waves (2 x 2) owns a BN x BM tile (weight rows x tokens).
 * Each 128-wide K step is one v_mfma_scale_f32_16x16x128_f8f6f4 per 16 x 16 sub-tile:
 * the weights are src A (fp4; lane (row r, q) holds the whole 32-wide block q, so the
 * row's E8M0 byte q is that lane's scale operand) and the activations src B (fp8).
 * Two activation modes:
 *   PF_A8  : e4m3 + one f32 scale per (token, 128 K) -- libref's quant_act_fp8 contract.
 *            Each MFMA runs with a unit activation scale on a zero accumulator; its result
 *            is multiplied by the token's step scale and added to the f32 accumulator,
 *            the per-group flush of libref's quant_dot (src/r3d_gemm_mxfp4.hip:263-300).
 *   PF_MX8 : e4m3 + one E8M0 per (token, 32 K) -- the mxfp8 activations of the bf16-in
 *            row.  Both scales ride in the MFMA, which accumulates in place.
 *
 * Staging: every byte a step needs arrives by direct global->LDS loads (16 bytes per lane
 * for the planes, 4 for the scales) into a three-deep ring, with one barrier per step.
 * Each 1 KB plane load fills exactly the LDS image of one MFMA operand fragment (lane l at
 * +16 l: 16 rows x 64 bytes of one step), so every fragment read is one contiguous
 * ds_read_b128 per lane, free of bank conflicts.  Weight rows past N and tokens past M
 * clamp to the last valid one; clamped lanes feed only outputs that are never stored.
 * Every load is unconditional (a step past the end reloads the last step into a ring slot
 * nobody reads), so the vmcnt bookkeeping is the same on every iteration.
 */
#ifndef R3D_PREFILL_H
#define R3D_PREFILL_H

#include "r3d_device.h"
#include "r3d_prefill_layout.h"

namespace r3d {

template <int MODE, int WNF, int WMF>
__global__ __launch_bounds__(256) void prefill_kernel(
    const uint8_t* __restrict__ A, const void* __restrict__ ASv,
    const uint8_t* __restrict__ B, const uint8_t* __restrict__ BS,
    uint16_t* __restrict__ Y,
    int M, int N, int steps, int grid_m, int tiles,
    int64_t a_pitch, int64_t as_pitch, int64_t b_pitch, int64_t bs_pitch, int64_t y_pitch) {
    using L = PrefillLayout<WNF, WMF, 3>;
    static_assert(WMF % 4 == 0, "activation fragments rotate through four register slots");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int li = lane & 15, q = lane >> 4;

    /* Workgroups go round-robin over the 8 XCDs; give each XCD a contiguous run of tiles,
     * token tiles fastest, so the workgroups sharing an L2 share weight and activation
     * tiles. */
    const int bid = blockIdx.x;
    const int per = tiles >> 3, rem = tiles & 7, x = bid & 7;
    const int t = x * per + (x < rem ? x : rem) + (bid >> 3);
    const int tm = t % grid_m, tn = t / grid_m;
    const int64_t n0 = (int64_t)tn * L::BN, m0 = (int64_t)tm * L::BM;

    /* ---- issue side.  Every source address is a wave-uniform tile base (advanced by one
     * K step per stage) plus a per-lane 32-bit offset fixed over K, so each direct load
     * is one VGPR offset on an SGPR base.  The host keeps 256 rows of any operand under
     * 2^31 bytes. */
    const uint8_t* const Bt = B + n0 * b_pitch;
    const uint8_t* const BSt = BS + n0 * bs_pitch;
    const uint8_t* const At = A + m0 * a_pitch;
    const int64_t xs_pitch = MODE == PF_MX8 ? as_pitch : 4 * as_pitch;     /* bytes */
    const uint8_t* const Xt = reinterpret_cast<const uint8_t*>(ASv) + m0 * xs_pitch;
    uint32_t woff[L::WLD];
#pragma unroll
    for (int i = 0; i < L::WLD; ++i) {
        const int f = wave + 4 * i;
        const int fr = f < L::WFR ? f : L::WFR - 1;         /* pad slots reload the last */
        int64_t n = n0 + 16 * fr + li;
        if (n > N - 1) n = N - 1;
        woff[i] = (uint32_t)((n - n0) * b_pitch + 16 * q);
    }
    uint32_t soff;
    {
        const int r = 64 * wave + lane < L::BN ? 64 * wave + lane : L::BN - 1;
        int64_t n = n0 + r;
        if (n > N - 1) n = N - 1;
        soff = (uint32_t)((n - n0) * bs_pitch);
    }
    uint32_t aoff[L::ALD];
#pragma unroll
    for (int i = 0; i < L::ALD; ++i) {
        const int j = wave + 4 * i;                          /* fragment j/2, half j%2 */
        int64_t m = m0 + 16 * (j >> 1) + li;
        if (m > M - 1) m = M - 1;
        aoff[i] = (uint32_t)((m - m0) * a_pitch + 64 * (j & 1) + 16 * q);
    }
    uint32_t xoff;
    {
        const int r = 64 * wave + lane < L::BM ? 64 * wave + lane : L::BM - 1;
        int64_t m = m0 + r;
        if (m > M - 1) m = M - 1;
        xoff = (uint32_t)((m - m0) * xs_pitch);
    }

    /* Direct load k (0 .. LOADS-1) of stage s into ring slot st: weight fragments, the
     * weight-scale dwords, activation half-fragments, the activation-scale dwords. */
    auto load = [&](int k, int s, uint8_t* st) {
        if (k < L::WLD) {
            r3d_lds_load(Bt + 64 * (int64_t)s + woff[k], st + L::W + 1024 * (wave + 4 * k), 16);
        } else if (k == L::WLD) {
            r3d_lds_load(BSt + 4 * (int64_t)s + soff, st + L::S + 256 * wave, 4);
        } else if (k < L::WLD + 1 + L::ALD) {
            const int i = k - L::WLD - 1;
            r3d_lds_load(At + 128 * (int64_t)s + aoff[i], st + L::A + 1024 * (wave + 4 * i), 16);
        } else {
            r3d_lds_load(Xt + 4 * (int64_t)s + xoff, st + L::AS + 256 * wave, 4);
        }
    };
    /* the loads of one stage, spread over the first WMF - 2 fragment groups of a step */
    constexpr int kParts = WMF - 2;
    constexpr int kPer = (L::LOADS + kParts - 1) / kParts;
    auto issue_part = [&](int part, int s, uint8_t* st) {
#pragma unroll
        for (int k = part * kPer; k < (part + 1) * kPer; ++k)
            if (k < L::LOADS) load(k, s, st);
    };

    /* ---- consume side: wave (wn, wm) owns WNF weight fragments x WMF token fragments.
     * Registers: two sets of weight fragments (this step's and the next's) and a ring of
     * four activation fragments, read two groups ahead. */
    const int wn = wave & 1, wm = wave >> 1;
    r3d_f32x4 acc[WNF][WMF];
#pragma unroll
    for (int a = 0; a < WNF; ++a)
#pragma unroll
        for (int b = 0; b < WMF; ++b) acc[a][b] = r3d_f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    r3d_i32x4 wA[WNF], wB[WNF];
    int xA[WNF], xB[WNF];
    r3d_i32x8 ar[4];
    int ax[4];
    float af[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    /* PF_A8: the MFMA results of the previous group, scaled and added one group later so
     * the VALU never waits on a result that is still in the matrix pipe */
    r3d_f32x4 dq[2][WNF];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int a = 0; a < WNF; ++a) dq[b][a] = r3d_f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    auto read_w = [&](const uint8_t* st, r3d_i32x4 (&w)[WNF], int (&xs)[WNF]) {
#pragma unroll
        for (int ni = 0; ni < WNF; ++ni) {
            const int f = wn * WNF + ni;
            w[ni] = *reinterpret_cast<const r3d_i32x4*>(st + L::W + 1024 * f + 16 * lane);
            xs[ni] = st[L::S + 4 * (16 * f + li) + q];
        }
    };
    auto read_a = [&](const uint8_t* st, int mi) {
        const int g = wm * WMF + mi, slot = mi & 3;
        const r3d_i32x4 lo = *reinterpret_cast<const r3d_i32x4*>(st + L::A + 2048 * g + 16 * lane);
        const r3d_i32x4 hi = *reinterpret_cast<const r3d_i32x4*>(st + L::A + 2048 * g + 1024 + 16 * lane);
        ar[slot] = r3d_i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        if (MODE == PF_MX8)
            ax[slot] = st[L::AS + 4 * (16 * g + li) + q];
        else
            af[slot] = *reinterpret_cast<const float*>(st + L::AS + 4 * (16 * g + li));
    };
    auto group = [&](int mi, const r3d_i32x4 (&w)[WNF], const int (&xs)[WNF]) {
        const int slot = mi & 3;
        if (MODE == PF_MX8) {
#pragma unroll
            for (int ni = 0; ni < WNF; ++ni)
                acc[ni][mi] = r3d_mfma_fp4_fp8_acc(w[ni], xs[ni], ar[slot], ax[slot], acc[ni][mi]);
        } else {
            const int pm = mi == 0 ? WMF - 1 : mi - 1;         /* the group flushed now */
            const float sp = af[(mi + 3) & 3];
#pragma unroll
            for (int ni = 0; ni < WNF; ++ni) {
                dq[mi & 1][ni] = r3d_mfma_fp4_fp8(w[ni], xs[ni], ar[slot], R3D_E8M0_ONE);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    acc[ni][pm][i] = acc[ni][pm][i] + dq[(mi + 1) & 1][ni][i] * sp;
            }
        }
    };
    /* One K step: stage s from ring slot cur, stage s + 2 loaded into slot fill, and --
     * after the step's barrier -- the first fragments of stage s + 1 read from slot nxt. */
    auto step = [&](int s, const uint8_t* cur, uint8_t* fill, const uint8_t* nxt,
                    const r3d_i32x4 (&wc)[WNF], const int (&xc)[WNF],
                    r3d_i32x4 (&wnx)[WNF], int (&xnx)[WNF]) {
        const int sf = s + 2 < steps ? s + 2 : steps - 1;
#pragma unroll
        for (int mi = 0; mi < WMF; ++mi) {
            group(mi, wc, xc);
            if (mi + 2 < WMF) {
                read_a(cur, mi + 2);
                issue_part(mi, sf, fill);
            } else if (mi + 2 == WMF) {
                /* every read of stage s is issued and stage s + 2 is in flight: wait for
                 * this wave's reads and for stage s + 1, then meet the other waves */
                asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" :: "n"(L::LOADS) : "memory");
                read_w(nxt, wnx, xnx);
                read_a(nxt, 0);
            } else {
                read_a(nxt, 1);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    /* ---- K walk */
    uint8_t* const st0 = smem;
    uint8_t* const st1 = smem + L::STAGE;
    uint8_t* const st2 = smem + 2 * L::STAGE;
#pragma unroll
    for (int k = 0; k < L::LOADS; ++k) load(k, 0, st0);
#pragma unroll
    for (int k = 0; k < L::LOADS; ++k) load(k, steps > 1 ? 1 : 0, st1);
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" :: "n"(L::LOADS) : "memory");
    read_w(st0, wA, xA);
    read_a(st0, 0);
    read_a(st0, 1);
    /* ring slots rotate 0 -> 1 -> 2 (stage s lives in slot s % 3); weight registers
     * alternate A / B, so the loop body is two steps */
    uint8_t* cur = st0;
    uint8_t* nxt = st1;
    uint8_t* fill = st2;
    for (int s = 0; s < steps; ++s) {
        step(s, cur, fill, nxt, wA, xA, wB, xB);
        uint8_t* t0 = cur; cur = nxt; nxt = fill; fill = t0;
#pragma unroll
        for (int ni = 0; ni < WNF; ++ni) { wA[ni] = wB[ni]; xA[ni] = xB[ni]; }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   /* drain the tail reloads */
    if (MODE == PF_A8) {
        /* the last group's results */
        const float sp = af[(WMF - 1) & 3];
#pragma unroll
        for (int ni = 0; ni < WNF; ++ni)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc[ni][WMF - 1][i] = acc[ni][WMF - 1][i] + dq[(WMF - 1) & 1][ni][i] * sp;
    }

    /* ---- epilogue: lane holds Y[m0 + 16 g + li][n0 + 16 f + 4 q + i], i = 0..3 */
    const bool vec = ((uintptr_t)Y & 7) == 0 && (y_pitch & 3) == 0;
#pragma unroll
    for (int ni = 0; ni < WNF; ++ni)
#pragma unroll
        for (int mi = 0; mi < WMF; ++mi) {
            const int64_t m = m0 + 16 * (wm * WMF + mi) + li;
            const int64_t n = n0 + 16 * (wn * WNF + ni) + 4 * q;
            if (m >= M || n >= N) continue;
            uint16_t* yp = Y + m * y_pitch + n;
            const r3d_f32x4 v = acc[ni][mi];
            if (vec && n + 3 < N) {
                const uint32_t lo = (uint32_t)r3d_bf16_rne(v[0]) | ((uint32_t)r3d_bf16_rne(v[1]) << 16);
                const uint32_t hi = (uint32_t)r3d_bf16_rne(v[2]) | ((uint32_t)r3d_bf16_rne(v[3]) << 16);
                *reinterpret_cast<uint2*>(yp) = make_uint2(lo, hi);
            } else {
                for (int i = 0; i < 4; ++i)
                    if (n + i < N) yp[i] = r3d_bf16_rne(v[i]);
            }
        }
}

/* ------------------------------------------------------------ mxfp8 quantiser -------
 * bf16 [M, K] -> e4m3 codes [M, K] + one E8M0 per 32 along K: the scale exponent is the
 * least e with amax * 2^-e <= 448 (clamped to [-127, 127]; 0 for an all-zero or
 * non-finite block), codes are x * 2^-e clamped to +-448 and rounded to nearest even.
 * Four lanes share a block (8 elements each, one 16-byte load); NaN elements never set
 * the block maximum and encode as 0x7F with their sign.  K % 32 == 0. */
__device__ __forceinline__ uint32_t r3d_e4m3_rne(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t s = (u >> 24) & 0x80u;
    const uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return s | 0x7Fu;
    if (a >= 0x43E00000u) return s | 0x7Eu;                    /* >= 448 */
    const int e = (int)(a >> 23) - 127;
    uint32_t m = a & 0x7FFFFFu;
    if (e < -10) return s;                                       /* below half the least subnormal */
    if (e < -6) {                                                /* e4m3 subnormal: m * 2^-9 */
        const int sh = 14 - e;
        m |= 0x800000u;
        const uint32_t lo = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
        uint32_t qq = m >> sh;
        if (lo > half || (lo == half && (qq & 1u))) ++qq;
        return s | qq;
    }
    uint32_t qq = m >> 20;
    const uint32_t lo = m & 0xFFFFFu;
    if (lo > 0x80000u || (lo == 0x80000u && (qq & 1u))) ++qq;
    int ee = e + 7;
    if (qq == 8u) { qq = 0; ++ee; }
    if (ee > 15 || (ee == 15 && qq >= 7u)) return s | 0x7Eu;
    return s | ((uint32_t)ee << 3) | qq;
}

__global__ __launch_bounds__(256) void quant_mx8_kernel(
    const uint16_t* __restrict__ X, int64_t x_pitch, uint8_t* __restrict__ Q, int64_t q_pitch,
    uint8_t* __restrict__ SX, int64_t sx_pitch, int64_t M, int K) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int per_row = K >> 3;
    const int64_t m = gid / per_row;
    const int c = (int)(gid - m * per_row);
    if (m >= M) return;                     /* whole 4-lane groups leave together */
    const r3d_i32x4 raw = *reinterpret_cast<const r3d_i32x4*>(X + m * x_pitch + 8 * c);
    float v[8];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float((uint32_t)raw[i] << 16);
        v[2 * i + 1] = __uint_as_float((uint32_t)raw[i] & 0xFFFF0000u);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float a = fabsf(v[i]);
        amax = a > amax ? a : amax;
    }
#pragma unroll
    for (int d = 1; d < 4; d <<= 1) {
        const float o = __shfl_xor(amax, d, 64);
        amax = o > amax ? o : amax;
    }
    int e = 0;
    const uint32_t ab = __float_as_uint(amax);
    if (ab != 0u && ab < 0x7F800000u) {
        const int bexp = (int)(ab >> 23);
        if (bexp == 0) {
            e = -127;                                      /* subnormal max: below any range */
        } else {
            /* amax = f * 2^ex, f in [0.5, 1): ex = bexp - 126; f > 0.875 <=> mantissa > 0.75 */
            const int ex = bexp - 126;
            e = (ab & 0x7FFFFFu) > 0x600000u ? ex - 8 : ex - 9;
            if (e < -127) e = -127;
            if (e > 127) e = 127;
        }
    }
    const float inv = (127 - e) >= 1 ? __uint_as_float((uint32_t)(127 - e) << 23)
                                     : __uint_as_float(0x00400000u);      /* 2^-127 */
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float cv = v[i] * inv;
        if (cv > 448.0f) cv = 448.0f;
        if (cv < -448.0f) cv = -448.0f;
        const uint32_t b = r3d_e4m3_rne(cv);
        if (i < 4) lo |= b << (8 * i);
        else hi |= b << (8 * (i - 4));
    }
    *reinterpret_cast<uint2*>(Q + m * q_pitch + 8 * c) = make_uint2(lo, hi);
    if ((threadIdx.x & 3) == 0) SX[m * sx_pitch + (c >> 2)] = (uint8_t)(e + 127);
}

}  // namespace r3d

#endif /* R3D_PREFILL_H */
