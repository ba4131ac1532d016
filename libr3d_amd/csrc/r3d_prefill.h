/* r3d_prefill.h -- the prefill GEMM of the mxfp4 gemm_nt_q rows on CDNA4 block-scaled
 * MFMA, and the bf16 -> mxfp8 activation quantiser that feeds its bf16-in row.
 *
 * Y[m, n] = sum_k A[m, k] * W[n, k], W in mxfp4 (e2m1 codes + one E8M0 per 32 along K),
 * A in e4m3.  A workgroup of 8 waves (2 along N x 4 along M, two per SIMD) owns a BN x BM
 * tile (weight rows x tokens).
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
 * Staging: every byte a step needs arrives by buffer loads straight into LDS (16 bytes
 * per lane for the planes, 4 for the scales) into a three-deep ring, with one barrier per
 * step; a stage is loaded the moment its slot frees, two steps ahead of its use.  Each 1 KB
 * plane load fills exactly the LDS image of one MFMA operand fragment
 * (16 rows x 64 bytes of one step, four lanes per row, XOR-swizzled), so every fragment
 * read is one ds_read_b128 per lane, free of bank conflicts.  Weight rows past N and
 * tokens past M clamp to the last valid one; clamped lanes feed only outputs that are
 * never stored.  Every load is unconditional (a step past the end reloads the last step
 * into a ring slot nobody reads), so the vmcnt bookkeeping is the same on every step.
 *
 * Register pipeline: activation fragments are read two groups ahead into a ring of four;
 * the weight fragments of step s + 1 are read into the second of two weight sets right
 * after step s's barrier (two groups before its end), which also releases the ring slot
 * just consumed for the load of stage s + 3.
 *
 * The mxfp8 MFMAs are issued through inline assembly with the accumulator tied to its
 * AGPRs ("+a"): it accumulates in place, and the register allocator cannot split the
 * accumulators' live ranges into copy chains.  Because the compiler then does not see
 * these MFMAs, each one carries its own s_nop 2 ahead of it (a VALU write of an operand
 * VGPR needs two wait states before an MFMA reads it), and the accumulators are read
 * after the loop only past 24 further wait states (an 8-pass MFMA result needs 11 before
 * a VALU or v_accvgpr_read may read it).  Nothing else writes an accumulator, and each
 * accumulator is rewritten only once per K step, dozens of MFMAs apart.
 */
#ifndef R3D_PREFILL_H
#define R3D_PREFILL_H

#include "r3d_band.h"
#include "r3d_device.h"
#include "r3d_prefill_layout.h"

namespace r3d {

/* acc += A(16 x 128 fp4, E8M0 scale per lane) . B(16 x 128 fp8, E8M0 scale per lane)^T,
 * in place in the accumulator's AGPRs (see the header comment for the hazard rules). */
__device__ __forceinline__ void r3d_mfma_mx_inplace(r3d_f32x4& acc, r3d_i32x4 a, int sa,
                                                    r3d_i32x8 b, int sb) {
    asm("s_nop 2\n\tv_mfma_scale_f32_16x16x128_f8f6f4 %0, %1, %2, %0, %3, %4 op_sel_hi:[0,0,0] cbsz:4 blgp:0"
        : "+a"(acc)
        : "v"(a), "v"(b), "v"(sa), "v"(sb));
}

template <int MODE, int WNF, int WMW, int WV = 8, int SBK = 0>
__global__ __launch_bounds__(64 * WV) void prefill_kernel(
    const uint8_t* __restrict__ A, const void* __restrict__ ASv,
    const uint8_t* __restrict__ B, const uint8_t* __restrict__ BS,
    uint16_t* __restrict__ Y,
    int M, int N, int ksteps, int grid_m, int tiles, int rblk,
    int64_t a_pitch, int64_t as_pitch, int64_t b_pitch, int64_t bs_pitch, int64_t y_pitch,
    int kc, int cst, float* __restrict__ part) {
    constexpr bool F8 = MODE == PF_F8;                   /* e4m3 weights, bf16 row scales */
    /* e4m3 weights on the 128 x 128 block grid (SBK): the tile's 128 weight rows share one
     * scale a K group, so the flush folds it into the token's scale first --
     * acc += D * (sa * sb), one fused multiply-add an element (libref rounds (D * sa) * sb;
     * the difference is one rounding of a product, inside the per-element bound) */
    constexpr bool SB = F8 && SBK;
    static_assert(!SB || 32 * WNF == 128, "one 128-row scale block a tile");
    constexpr int WH = F8 ? 2 : 1;                        /* 1 KB images per weight fragment */
    constexpr int WB = 64 * WH;                           /* weight bytes per row per step */
    using L = PrefillLayout<WNF, WMW, 3, WH, WV>;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);     /* 0 .. WV-1 */
    const int li = lane & 15, q = lane >> 4;

    /* The grid is tiles x kc units: unit u is K chunk u / tiles (steps [cst c, cst c + cst)
     * of the K walk, clipped to ksteps) of tile u % tiles.  kc = 1 is the whole K walk.
     * Workgroups go round-robin over the 8 XCDs; give each XCD a contiguous run of units,
     * so the workgroups sharing an L2 share weight and activation tiles (and, split, one
     * chunk's activation columns).  Tiles run in groups of 8 weight tiles: token tile
     * major, weight tile fastest inside a group, so one round of 32 workgroups on an XCD
     * covers 8 weight x 4 token tiles (config 3: 10.3 MB of panels a round against 13.4 MB
     * for 4 x 8; measured 1-1.5 % faster). */
    /* the split runs on the tiles of up to 128 tokens of the flushed modes only; the other
     * instantiations compile it out (it costs them registers) and take kc = 1 */
    constexpr bool KS = MODE != PF_MX8 && WMW <= 2 && WV == 8;
    const int bid = blockIdx.x;
    const int units = KS ? tiles * kc : tiles;
    const int per = units >> 3, rem = units & 7, x = bid & 7;
    const int u = x * per + (x < rem ? x : rem) + (bid >> 3);
    const int kci = KS ? u / tiles : 0, t = u - kci * tiles;
    const int64_t s0 = (int64_t)kci * cst;             /* first K step of the chunk */
    const int steps = !KS ? ksteps : ksteps - (int)s0 < cst ? ksteps - (int)s0 : cst;
    int tm, tn;
    {
        constexpr int GN = 8;
        const int grid_n = tiles / grid_m;
        const int grp = t / (GN * grid_m), in = t - grp * GN * grid_m, gn0 = grp * GN;
        const int gw = grid_n - gn0 < GN ? grid_n - gn0 : GN;     /* the last group's width */
        tm = in / gw;
        tn = gn0 + (in - tm * gw);
    }
    const int64_t n0 = (int64_t)tn * L::BN, m0 = (int64_t)tm * L::BM;

    /* ---- issue side: one buffer resource per operand, based at this tile's first row and
     * bounded by the operand's end; per-lane 32-bit offsets fixed over K; the K step
     * rides in the scalar offset.  The host keeps 256 rows of any operand under 2^31
     * bytes. */
    const int64_t xs_pitch = MODE == PF_MX8 ? as_pitch : 4 * as_pitch;     /* bytes */
    /* a chunk starts s0 steps into every row: WB weight bytes, 128 activation bytes, one
     * weight scale dword (e4m3 weights: one bf16) and one activation scale dword a step */
    const int64_t wk = WB * s0, ak = 128 * s0, wsk = (F8 ? 2 : 4) * s0, ask = 4 * s0;
    const __amdgpu_buffer_rsrc_t rB = r3d_rsrc(B + n0 * b_pitch + wk, (N - n0) * b_pitch - wk);
    const __amdgpu_buffer_rsrc_t rA = r3d_rsrc(A + m0 * a_pitch + ak, (M - m0) * a_pitch - ak);
    /* scales: at 8 waves, waves 0-3 fetch the weight rows' scales (E8M0 dwords; e4m3
     * weights: the bf16 of the row's scale row n / rblk), waves 4-7 the tokens'; at 4 waves
     * every wave fetches 64 of each (wsc: this wave's first scale load is the weights') */
    const bool wsc = WV == 4 || wave < 4;
    const int64_t sr0 = F8 ? n0 / rblk : n0;             /* first scale row of the tile */
    const int64_t srn = F8 ? (N - 1) / rblk + 1 : N;     /* scale rows */
    const int64_t ws_pitch = F8 ? 2 * bs_pitch : bs_pitch;    /* bytes */
    const __amdgpu_buffer_rsrc_t rSX =
        wsc ? r3d_rsrc(BS + sr0 * ws_pitch + wsk, (srn - sr0) * ws_pitch - wsk)
            : r3d_rsrc(reinterpret_cast<const uint8_t*>(ASv) + m0 * xs_pitch + ask,
                       (M - m0) * xs_pitch - ask);
    /* A plane load covers 16 rows x 64 bytes with four consecutive lanes on each row
     * (lane l: row l / 4), so every row is one 64-byte run; chunk l % 4 of the run is
     * fetched XOR-swizzled by (row / 2) % 4.  An MFMA operand read (row li, chunk q) then
     * sits at 16-byte position 4 li + (q ^ (li / 2) % 4), and any 8 consecutive lanes --
     * one 128-byte LDS cycle of a ds_read_b128 -- hit 8 distinct bank groups. */
    const int lr = lane >> 2;                                /* row of this lane's load */
    const int lc = (lane & 3) ^ ((lr >> 1) & 3);             /* chunk it fetches */
    uint32_t woff[L::WLD];
#pragma unroll
    for (int i = 0; i < L::WLD; ++i) {
        /* image j: fragment j / WH, 64-byte half j % WH (e4m3 rows are two halves) */
        const int j = wave + WV * i;
        const int jr = j < WH * L::WFR ? j : WH * L::WFR - 1;    /* pad slots reload the last */
        int64_t n = n0 + 16 * (jr / WH) + lr;
        if (n > N - 1) n = N - 1;
        woff[i] = (uint32_t)((n - n0) * b_pitch + 64 * (jr % WH) + 16 * lc);
    }
    uint32_t sxoff;
    {
        const int r0 = 64 * (wave & 3) + lane;
        if (wsc) {
            int64_t n = n0 + (r0 < L::BN ? r0 : L::BN - 1);
            if (n > N - 1) n = N - 1;
            sxoff = (uint32_t)(((F8 ? n / rblk : n) - sr0) * ws_pitch);
        } else {
            int64_t m = m0 + (r0 < L::BM ? r0 : L::BM - 1);
            if (m > M - 1) m = M - 1;
            sxoff = (uint32_t)((m - m0) * xs_pitch);
        }
    }
    const int sxdst = (wsc ? L::S : L::AS) + 256 * (wave & 3);
    /* 4 waves: the tokens' scales are each wave's second scale load */
    const __amdgpu_buffer_rsrc_t rSA =
        r3d_rsrc(reinterpret_cast<const uint8_t*>(ASv) + m0 * xs_pitch + ask,
                 (M - m0) * xs_pitch - ask);
    uint32_t saoff;
    {
        const int r0 = 64 * (wave & 3) + lane;
        int64_t m = m0 + (r0 < L::BM ? r0 : L::BM - 1);
        if (m > M - 1) m = M - 1;
        saoff = (uint32_t)((m - m0) * xs_pitch);
    }
    const int sadst = L::AS + 256 * (wave & 3);
    uint32_t aoff[L::ALD];
#pragma unroll
    for (int i = 0; i < L::ALD; ++i) {
        const int j = wave + WV * i;                         /* fragment j/2, half j%2 */
        int64_t m = m0 + 16 * (j >> 1) + lr;
        if (m > M - 1) m = M - 1;
        aoff[i] = (uint32_t)((m - m0) * a_pitch + 64 * (j & 1) + 16 * lc);
    }
    /* load k (0 .. LOADS-1) of stage s into ring slot st */
    auto load = [&](int k, int s, uint8_t* st) __attribute__((always_inline)) {
        if (k < L::WLD)
            r3d_buf_lds<16>(rB, st + L::W + 1024 * (wave + WV * k), woff[k], WB * s);
        else if (k == L::WLD && F8 && wsc)
            r3d_buf_lds<2>(rSX, st + sxdst, sxoff, 2 * s);        /* one bf16 per weight row */
        else if (k == L::WLD)
            r3d_buf_lds<4>(rSX, st + sxdst, sxoff, 4 * s);
        else if (WV == 4 && k == L::WLD + 1)
            r3d_buf_lds<4>(rSA, st + sadst, saoff, 4 * s);        /* the tokens' scales */
        else
            r3d_buf_lds<16>(rA, st + L::A + 1024 * (wave + WV * (k - L::WLD - L::SLD)),
                            aoff[k - L::WLD - L::SLD], 128 * s);
    };
    /* a stage's loads go out in WMW parts, one per fragment group, so the load issue
     * never stalls a wave for a whole stage at once */
    constexpr int kPer = (L::LOADS + WMW - 1) / WMW;
    auto issue_part = [&](int part, int s, uint8_t* st) __attribute__((always_inline)) {
        const int sc = s < steps ? s : steps - 1;
#pragma unroll
        for (int k = part * kPer; k < (part + 1) * kPer; ++k)
            if (k < L::LOADS) load(k, sc, st);
    };

    /* ---- consume side: wave (wn, wm) owns WNF weight fragments x WMW token fragments.
     * Two weight sets (this step's and the next's) and a ring of four activation
     * fragments read two groups ahead. */
    const int wn = wave & 1, wm = wave >> 1;
    r3d_f32x4 acc[WNF][WMW];
#pragma unroll
    for (int a = 0; a < WNF; ++a)
#pragma unroll
        for (int b = 0; b < WMW; ++b) acc[a][b] = r3d_f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    r3d_i32x4 wS[2][WNF];
    int xS[2][WNF];
    /* PF_F8: the e4m3 weight operands and, per fragment, the bf16 scales (4-byte slots) of
     * the lane's four result rows 4q .. 4q + 3; zero until the first step's are read, so
     * the first (empty) deferred flush multiplies zeros */
    /* e4m3 weights on the single-operand-set walk (SS below) */
    constexpr bool SSF = F8 && (WMW == 4 || WMW == 8);
    r3d_i32x8 wF[2][WNF];
    r3d_i32x4 sbF[2][WNF];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int a = 0; a < WNF; ++a) sbF[b][a] = r3d_i32x4{0, 0, 0, 0};
    /* the single-operand-set walk (SS below) holds the same bf16 scales two to a register:
     * rows 4q, 4q + 1 in word 0 (low, high half), rows 4q + 2, 4q + 3 in word 1 */
    uint32_t sbP[2][WNF][2];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int a = 0; a < WNF; ++a) sbP[b][a][0] = sbP[b][a][1] = 0u;
    auto pack_sb = [&](const uint8_t* src, int set, int ni) __attribute__((always_inline)) {
        const r3d_i32x4 v = *reinterpret_cast<const r3d_i32x4*>(src);
        /* bytes 0-1 of v[0] then bytes 0-1 of v[1] (v_perm_b32: selector bytes 0-3 pick
         * the second source, 4-7 the first) */
        sbP[set][ni][0] = __builtin_amdgcn_perm((uint32_t)v[1], (uint32_t)v[0], 0x05040100u);
        sbP[set][ni][1] = __builtin_amdgcn_perm((uint32_t)v[3], (uint32_t)v[2], 0x05040100u);
    };
    /* SB: the tile's block scale of each weight set (every row's slot holds it; slot 0) */
    float sbB[2] = {0.0f, 0.0f};
    auto read_sb = [&](const uint8_t* st, int set) __attribute__((always_inline)) {
        sbB[set] = __uint_as_float((uint32_t)*reinterpret_cast<const uint16_t*>(st + L::S) << 16);
    };
    r3d_i32x8 ar[4];
    int ax[4];
    float af[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float sprev = 0.0f;
    /* PF_A8: the MFMA results of the previous group, scaled and added one group later so
     * the VALU never waits on a result that is still in the matrix pipe */
    r3d_f32x4 dq[2][WNF];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int a = 0; a < WNF; ++a) dq[b][a] = r3d_f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    /* this lane's operand chunk (row li, chunk q) inside any 1 KB fragment image */
    const int rd = 16 * (4 * li + (q ^ ((li >> 1) & 3)));
    auto read_w = [&](const uint8_t* st, int set) __attribute__((always_inline)) {
#pragma unroll
        for (int ni = 0; ni < WNF; ++ni) {
            const int f = wn * WNF + ni;
            if (F8) {
                const r3d_i32x4 lo = *reinterpret_cast<const r3d_i32x4*>(st + L::W + 2048 * f + rd);
                const r3d_i32x4 hi =
                    *reinterpret_cast<const r3d_i32x4*>(st + L::W + 2048 * f + 1024 + rd);
                wF[set][ni] = r3d_i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                if (SB) {
                    if (ni == 0) read_sb(st, set);
                } else if (SSF) {
                    pack_sb(st + L::S + 4 * (16 * f + 4 * q), set, ni);
                } else {
                    sbF[set][ni] = *reinterpret_cast<const r3d_i32x4*>(st + L::S + 4 * (16 * f + 4 * q));
                }
            } else {
                wS[set][ni] = *reinterpret_cast<const r3d_i32x4*>(st + L::W + 1024 * f + rd);
                xS[set][ni] = st[L::S + 4 * (16 * f + li) + q];
            }
        }
    };
    auto read_a = [&](const uint8_t* st, int mi) __attribute__((always_inline)) {
        const int g = wm * WMW + mi, slot = mi & 3;
        const r3d_i32x4 lo = *reinterpret_cast<const r3d_i32x4*>(st + L::A + 2048 * g + rd);
        const r3d_i32x4 hi = *reinterpret_cast<const r3d_i32x4*>(st + L::A + 2048 * g + 1024 + rd);
        ar[slot] = r3d_i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        if (MODE == PF_MX8)
            ax[slot] = st[L::AS + 4 * (16 * g + li) + q];
        else
            af[slot] = *reinterpret_cast<const float*>(st + L::AS + 4 * (16 * g + li));
    };
    /* one token group a wave (the split tiles): a wave whose 16 tokens all lie past M
     * (clamped padding rows, never stored) skips its MFMAs; its flushes still run, on stale
     * results into accumulators that are never stored.  (Wider tiles issue every MFMA: the
     * branch costs them registers.) */
    const int mlive = WMW == 1 && 16 * (int64_t)wm >= M - m0 ? 0 : WMW;
    /* the result pair dq[2] alternates group by group along the whole K walk: by the group
     * index at an even group count a step, also by the step (the weight set) at an odd one */
    auto group = [&](int mi, int set) __attribute__((always_inline)) {
        const int slot = mi & 3;
        const bool live = mi < mlive;
        const int dc = ((WMW & 1) ? set : 0) ^ (mi & 1), dp = dc ^ 1;
        if (MODE == PF_MX8) {
            if (live) {
#pragma unroll
                for (int ni = 0; ni < WNF; ++ni)
                    r3d_mfma_mx_inplace(acc[ni][mi], wS[set][ni], xS[set][ni], ar[slot], ax[slot]);
            }
        } else if (F8) {
            /* libref's (sub * sa) * sb flush (src/r3d_gemm_fp8a8.hip:9-15), deferred one
             * group; the flushed group of group 0 is the previous step's last, whose weight
             * scales are still in the other set (it is refilled only after this group) */
            const int pm = mi == 0 ? WMW - 1 : mi - 1;
            const int ps = mi == 0 ? set ^ 1 : set;
#pragma unroll
            for (int ni = 0; ni < WNF; ++ni) {
                if (live) dq[dc][ni] = r3d_mfma_fp8_fp8(wF[set][ni], ar[slot]);
                if (SB) {
                    const float sf = sprev * sbB[ps];
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        acc[ni][pm][i] = __builtin_fmaf(dq[dp][ni][i], sf, acc[ni][pm][i]);
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float sb = __uint_as_float((uint32_t)sbF[ps][ni][i] << 16);
                        acc[ni][pm][i] = acc[ni][pm][i] + (dq[dp][ni][i] * sprev) * sb;
                    }
                }
            }
            sprev = af[slot];
        } else {
            const int pm = mi == 0 ? WMW - 1 : mi - 1;         /* the group flushed now */
#pragma unroll
            for (int ni = 0; ni < WNF; ++ni) {
                if (live)
                    dq[dc][ni] = r3d_mfma_fp4_fp8(wS[set][ni], xS[set][ni], ar[slot], R3D_E8M0_ONE);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    acc[ni][pm][i] = acc[ni][pm][i] + dq[dp][ni][i] * sprev;
            }
            sprev = af[slot];        /* this group's scale, kept past the slot's refill */
        }
    };
    /* Flushed modes (PF_A8, PF_F8) with four (or eight) token fragments per wave: ONE weight operand
     * set -- fragment ni of step s + 1 is read into it right after the last group's MFMA on
     * fragment ni of step s, WNF MFMAs before its first use -- and the MFMA results in a
     * ring of RR, each flushed LAG MFMAs after its issue (past the result latency), so the
     * registers of a second weight set and of two whole result sets go to the larger tile.
     * The flush of MFMA t (index mi * WNF + ni in the step) uses its group's a_scale: the
     * current group's, or sprev for the group before (the previous step's last group at
     * mi = 0), and at e4m3 weights the row scales of its step's set. */
    constexpr bool SS = MODE != PF_MX8 && (WMW == 4 || WMW == 8);
    constexpr int RR = 4, LAG = RR - 1;
    static_assert(!SS || ((WMW * WNF) % RR == 0 && LAG < WNF), "result ring period");
    r3d_f32x4 dqr[RR];
#pragma unroll
    for (int r = 0; r < RR; ++r) dqr[r] = r3d_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    auto read_w1 = [&](const uint8_t* st, int ni, int sset) __attribute__((always_inline)) {
        const int f = wn * WNF + ni;
        if (F8) {
            const r3d_i32x4 lo = *reinterpret_cast<const r3d_i32x4*>(st + L::W + 2048 * f + rd);
            const r3d_i32x4 hi = *reinterpret_cast<const r3d_i32x4*>(st + L::W + 2048 * f + 1024 + rd);
            wF[0][ni] = r3d_i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            if (SB) {
                if (ni == 0) read_sb(st, sset);
            } else {
                pack_sb(st + L::S + 4 * (16 * f + 4 * q), sset, ni);
            }
        } else {
            wS[0][ni] = *reinterpret_cast<const r3d_i32x4*>(st + L::W + 1024 * f + rd);
            xS[0][ni] = st[L::S + 4 * (16 * f + li) + q];
        }
    };
    auto flush1 = [&](int t, int mi, float scur, int set) __attribute__((always_inline)) {
        const bool before = t < 0;                      /* the previous step's last group */
        const int tt = before ? t + WMW * WNF : t;
        const int nf = tt % WNF, mf = tt / WNF;
        const float sv = (!before && mf == mi) ? scur : sprev;
        const r3d_f32x4 d = dqr[tt % RR];
        const float sf = SB ? sv * (before ? sbB[set ^ 1] : sbB[set]) : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (SB) {
                acc[nf][mf][i] = __builtin_fmaf(d[i], sf, acc[nf][mf][i]);
            } else if (F8) {
                const uint32_t pw = before ? (set ? sbP[0][nf][i >> 1] : sbP[1][nf][i >> 1])
                                           : (set ? sbP[1][nf][i >> 1] : sbP[0][nf][i >> 1]);
                const float sb = __uint_as_float((i & 1) ? (pw & 0xFFFF0000u) : (pw << 16));
                acc[nf][mf][i] = acc[nf][mf][i] + (d[i] * sv) * sb;
            } else {
                acc[nf][mf][i] = acc[nf][mf][i] + d[i] * sv;
            }
        }
    };
    auto group1 = [&](int mi, int set, const uint8_t* nxt) __attribute__((always_inline)) {
        const int slot = mi & 3;
        const float scur = af[slot];
#pragma unroll
        for (int ni = 0; ni < WNF; ++ni) {
            const int t = mi * WNF + ni;
            if (F8)
                dqr[t % RR] = r3d_mfma_fp8_fp8(wF[0][ni], ar[slot]);
            else
                dqr[t % RR] = r3d_mfma_fp4_fp8(wS[0][ni], xS[0][ni], ar[slot], R3D_E8M0_ONE);
            if (mi == WMW - 1) read_w1(nxt, ni, set ^ 1);
            flush1(t - LAG, mi, scur, set);
        }
        sprev = scur;
    };
    auto step_ss = [&](int s, int set, uint8_t* cur, const uint8_t* nxt, uint8_t* prv) __attribute__((always_inline)) {
#pragma unroll
        for (int mi = 0; mi < WMW; ++mi) {
            group1(mi, set, nxt);
            if (mi + 2 < WMW) {
                read_a(cur, mi + 2);
                issue_part(mi + 2, s + 2, prv);
            } else if (mi + 2 == WMW) {
                asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" :: "n"(L::LOADS) : "memory");
                issue_part(0, s + 3, cur);
                read_a(nxt, 0);
            } else {
                issue_part(1, s + 3, cur);
                read_a(nxt, 1);
            }
#ifdef R3D_PF_SCHED
            if (F8) {
                __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);    /* the group's LDS reads */
#pragma unroll
                for (int k = 0; k < WNF; ++k) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, R3D_PF_SCHED, 0);
                }
            }
#endif
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    /* One K step on weight set `set` from ring slot cur (stage s); nxt and prv are the
     * slots of stages s + 1 and s - 1 (= s + 2).  At group WMW - 2 every read of stage s
     * has been issued: once this wave's reads are done and stage s + 1 has landed, the
     * barrier releases slot cur for stage s + 3, and the first fragments of stage s + 1
     * are read from slot nxt into the other weight set.  Stage k's loads go out in the
     * WMW groups between the barriers of steps k - 3 and k - 2, so at each barrier exactly
     * one stage (LOADS loads) is younger than the one it waits for. */
    auto step = [&](int s, int set, uint8_t* cur, const uint8_t* nxt, uint8_t* prv) __attribute__((always_inline)) {
        if (SS) { step_ss(s, set, cur, nxt, prv); return; }
        if (WMW == 1) {
            /* one token group: its MFMAs, then the barrier, stage s + 3 whole into the slot
             * just released, and stage s + 1's fragments (stage s + 2 went out a step ago,
             * so the wait leaves exactly one stage in flight, as below) */
            group(0, set);
            asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" :: "n"(L::LOADS) : "memory");
            issue_part(0, s + 3, cur);
            read_w(nxt, set ^ 1);
            read_a(nxt, 0);
            __builtin_amdgcn_sched_barrier(0);
            return;
        }
#pragma unroll
        for (int mi = 0; mi < WMW; ++mi) {
            group(mi, set);
            if (mi + 2 < WMW) {
                read_a(cur, mi + 2);
                issue_part(mi + 2, s + 2, prv);
            } else if (mi + 2 == WMW) {
                asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" :: "n"(L::LOADS) : "memory");
                issue_part(0, s + 3, cur);
                read_w(nxt, set ^ 1);
                read_a(nxt, 0);
            } else {
                issue_part(1, s + 3, cur);
                read_a(nxt, 1);
            }
            /* keep each group's reads and loads beside its own MFMAs */
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    /* ---- K walk: stage s lives in ring slot s % 3 and weight set s % 2 */
#pragma unroll
    for (int p = 0; p < WMW; ++p) issue_part(p, 0, smem);
#pragma unroll
    for (int p = 0; p < WMW; ++p) issue_part(p, 1, smem + L::STAGE);
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" :: "n"(L::LOADS) : "memory");
    issue_part(0, 2, smem + 2 * L::STAGE);
    issue_part(1, 2, smem + 2 * L::STAGE);
    read_w(smem, 0);
    read_a(smem, 0);
    if (WMW > 1) read_a(smem, 1);
    int sl = 0;                                         /* ring slot of stage s */
    int s = 0;
    /* e4m3 weights on the single-operand-set walk: six steps an iteration (the period of
     * three ring slots and two weight sets), so every slot's LDS address is a constant and
     * the reads take immediate offsets instead of per-read address arithmetic; the same
     * steps in the same order as the two-step loop below, which takes the rest */
    constexpr bool U6 = SS && F8;
    if (U6) {
        uint8_t* const r0 = smem;
        uint8_t* const r1 = smem + L::STAGE;
        uint8_t* const r2 = smem + 2 * L::STAGE;
        for (; s + 6 <= steps; s += 6) {
            step(s, 0, r0, r1, r2);
            step(s + 1, 1, r1, r2, r0);
            step(s + 2, 0, r2, r0, r1);
            step(s + 3, 1, r0, r1, r2);
            step(s + 4, 0, r1, r2, r0);
            step(s + 5, 1, r2, r0, r1);
        }
    }
    for (; s + 2 <= steps; s += 2) {
        const int s1 = sl == 2 ? 0 : sl + 1, s2 = s1 == 2 ? 0 : s1 + 1;
        step(s, 0, smem + sl * L::STAGE, smem + s1 * L::STAGE, smem + s2 * L::STAGE);
        step(s + 1, 1, smem + s1 * L::STAGE, smem + s2 * L::STAGE, smem + sl * L::STAGE);
        sl = s2;
    }
    if (s < steps) {
        const int s1 = sl == 2 ? 0 : sl + 1, s2 = s1 == 2 ? 0 : s1 + 1;
        step(s, 0, smem + sl * L::STAGE, smem + s1 * L::STAGE, smem + s2 * L::STAGE);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   /* drain the tail reloads */
    if (MODE == PF_MX8) {
        /* 24 wait states between the last in-place MFMA and any read of an accumulator;
         * the empty statements order every read after them */
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
        for (int a = 0; a < WNF; ++a)
#pragma unroll
            for (int b = 0; b < WMW; ++b) asm volatile("" : "+a"(acc[a][b]));
    } else if (SS) {
        /* the last LAG results of the last step (its last group; sprev is its scale) */
        const int ls = (steps - 1) & 1;
#pragma unroll
        for (int t = WMW * WNF - LAG; t < WMW * WNF; ++t) flush1(t, WMW - 1, sprev, ls);
    } else {
        /* the last group's results (at e4m3 weights with the last step's weight set's
         * scales: steps alternate sets starting from set 0; at one group a step its result
         * pair alternates the same way) */
        const int ls = (steps - 1) & 1;
#pragma unroll
        for (int ni = 0; ni < WNF; ++ni)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float d = (WMW & 1) ? ((ls ^ ((WMW - 1) & 1)) ? dq[1][ni][i] : dq[0][ni][i])
                                          : dq[(WMW - 1) & 1][ni][i];
                if (SB) {
                    acc[ni][WMW - 1][i] = __builtin_fmaf(d, sprev * (ls ? sbB[1] : sbB[0]),
                                                         acc[ni][WMW - 1][i]);
                } else if (F8) {
                    const uint32_t sbb = (uint32_t)(ls ? sbF[1][ni][i] : sbF[0][ni][i]);
                    const float sb = __uint_as_float(sbb << 16);
                    acc[ni][WMW - 1][i] = acc[ni][WMW - 1][i] + (d * sprev) * sb;
                } else {
                    acc[ni][WMW - 1][i] = acc[ni][WMW - 1][i] + d * sprev;
                }
            }
    }

    /* ---- split K: the f32 partial tile goes to plane kci of part ([kc][M][N], 16-byte
     * aligned), four consecutive columns a lane */
    if (KS && part) {
        /* every accumulator complete in every lane before the lane-divergent stores (the
         * compiler may otherwise sink the last MFMAs into them, where lanes off the exec
         * mask would hand the MFMA stale operands) */
#pragma unroll
        for (int ni = 0; ni < WNF; ++ni)
#pragma unroll
            for (int mi = 0; mi < WMW; ++mi) asm volatile("" : "+v"(acc[ni][mi]));
        float* pp = part + (int64_t)kci * M * N;
        const bool v4 = (N & 3) == 0;
#pragma unroll
        for (int ni = 0; ni < WNF; ++ni)
#pragma unroll
            for (int mi = 0; mi < WMW; ++mi) {
                const int64_t m = m0 + 16 * (wm * WMW + mi) + li;
                const int64_t n = n0 + 16 * (wn * WNF + ni) + 4 * q;
                if (m >= M || n >= N) continue;
                const r3d_f32x4 v = acc[ni][mi];
                float* d = pp + m * N + n;
                if (v4) {
                    *reinterpret_cast<r3d_f32x4*>(d) = v;
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (n + i < N) d[i] = v[i];
                }
            }
        return;
    }

    /* ---- epilogue: lane holds Y[m0 + 16 g + li][n0 + 16 f + 4 q + i], i = 0..3.  The bf16
     * tile is staged through the (now idle) LDS ring and leaves as whole 16-byte row chunks,
     * so every store instruction writes full contiguous row segments.  LDS row pitch: 2 BN
     * bytes padded to 32 mod 128, so the 16 lanes of one 8-byte write cycle (4 rows x 4
     * column chunks) cover 32 distinct banks. */
    constexpr int YP = 2 * L::BN + (32 - (2 * L::BN) % 128 + 128) % 128;
    constexpr int CPR = L::BN / 8;                     /* 16-byte chunks per tile row */
    static_assert(L::BM * YP <= L::LDS, "the output tile fits the ring");
    __syncthreads();                                   /* every wave is done with the ring */
#pragma unroll
    for (int ni = 0; ni < WNF; ++ni)
#pragma unroll
        for (int mi = 0; mi < WMW; ++mi) {
            const int ml = 16 * (wm * WMW + mi) + li;
            const int nl = 16 * (wn * WNF + ni) + 4 * q;
            const r3d_f32x4 v = acc[ni][mi];
            *reinterpret_cast<uint2*>(smem + ml * YP + 2 * nl) =
                make_uint2(r3d_pack_bf16x2(v[0], v[1]), r3d_pack_bf16x2(v[2], v[3]));
        }
    __syncthreads();
    const bool vec = ((uintptr_t)Y & 15) == 0 && (y_pitch & 7) == 0;
    for (int e = threadIdx.x; e < L::BM * CPR; e += 64 * L::WAVES) {
        const int r = e / CPR, c = e - (e / CPR) * CPR;
        const int64_t m = m0 + r, n = n0 + 8 * c;
        if (m >= M || n >= N) continue;
        const r3d_i32x4 v = *reinterpret_cast<const r3d_i32x4*>(smem + r * YP + 16 * c);
        uint16_t* yp = Y + m * y_pitch + n;
        if (vec && n + 8 <= N) {
            *reinterpret_cast<r3d_i32x4*>(yp) = v;
        } else {
            const uint16_t* h = reinterpret_cast<const uint16_t*>(&v);
            for (int i = 0; i < 8; ++i)
                if (n + i < N) yp[i] = h[i];
        }
    }
}

/* Split K's second kernel: Y[m, n] = bf16(sum over c = 0 .. kc-1 of part[c][m][n]), the
 * chunks added in order from +0 (so every call sums the same way), four columns a lane.
 * BATCH chunk loads go out together ahead of their adds; TH lanes a workgroup.  A
 * decode-sized Y (a few thousand lanes) takes <64, 16>: its planes, written by the kernel
 * just before on other CUs, are read from memory once for up to 16 chunks, over many CUs
 * (C2 down at M = 4: the split call 15.80 -> 15.48 us).  A larger Y (M = 16..64) has the
 * lanes to hide the latency and keeps <256, 4>, whose fewer registers a lane measured
 * 1-2 % faster there. */
template <int TH, int BATCH>
__global__ __launch_bounds__(TH) void splitk_reduce_kernel(
    const float* __restrict__ part, int kc, int M, int N, uint16_t* __restrict__ Y,
    int64_t y_pitch) {
    /* grid: (column quads / TH, M rows) -- the row is the workgroup's y index, so no lane
     * divides by the row length before its first load */
    const int cpr = (N + 3) >> 2;
    const int q = blockIdx.x * TH + threadIdx.x;
    if (q >= cpr) return;
    const int m = blockIdx.y, n = 4 * q;
    const int64_t plane = (int64_t)M * N;
    const float* p = part + (int64_t)m * N + n;
    r3d_f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
    if ((N & 3) == 0) {
        for (int c = 0; c < kc; c += BATCH) {
            r3d_f32x4 v[BATCH];
#pragma unroll
            for (int j = 0; j < BATCH; ++j)
                if (c + j < kc) v[j] = *reinterpret_cast<const r3d_f32x4*>(p + (c + j) * plane);
#pragma unroll
            for (int j = 0; j < BATCH; ++j)
                if (c + j < kc) s += v[j];
        }
    } else {
        for (int c = 0; c < kc; ++c)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (n + i < N) s[i] += p[c * plane + i];
    }
    uint16_t* yp = Y + m * y_pitch + n;
    const uint32_t lo = r3d_pack_bf16x2(s[0], s[1]), hi = r3d_pack_bf16x2(s[2], s[3]);
    if (((uintptr_t)yp & 7) == 0 && n + 4 <= N) {
        *reinterpret_cast<uint2*>(yp) = make_uint2(lo, hi);
    } else {
        const uint16_t h[4] = {(uint16_t)lo, (uint16_t)(lo >> 16), (uint16_t)hi, (uint16_t)(hi >> 16)};
        for (int i = 0; i < 4; ++i)
            if (n + i < N) yp[i] = h[i];
    }
}

/* ------------------------------------------------------------ mxfp8 quantiser -------
 * bf16 [M, K] -> e4m3 codes [M, K] + one E8M0 per 32 along K: the scale exponent is the
 * least e with amax * 2^-e <= 448 (clamped to [-127, 127]; 0 for an all-zero or
 * non-finite block), codes are x * 2^-e clamped to +-448 and rounded to nearest even.
 * NaN elements never set the block maximum and encode as 0x7F with their sign. */
/* f32 -> e4m3 code, round to nearest even, saturating at +-448, NaN -> 0x7F with the sign.
 * Branch-free (selects only): on MI355X it gives the same code as the step-by-step form
 * (exponent / mantissa split, explicit subnormal shift and tie test) for every one of the
 * 2^32 inputs after the quantiser's +-448 clamp (checked exhaustively on the device); the
 * kernels encode with r3d_e4m3x4_rne (r3d_band.h), checked equal to it on all inputs. */
__device__ __forceinline__ uint32_t r3d_e4m3_rne(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t s = (u >> 24) & 0x80u;
    const uint32_t a = u & 0x7FFFFFFFu;
    /* normal range: exponent field, top 3 mantissa bits, nearest-even on the other 20; a
     * carry out of the mantissa moves into the exponent through the plain add */
    const uint32_t m = a & 0x7FFFFFu;
    const uint32_t lo = m & 0xFFFFFu;
    const uint32_t rnd = (lo > 0x80000u) | ((lo == 0x80000u) & (m >> 20) & 1u);
    const uint32_t nrm = ((((a >> 23) - 120u) << 3) | (m >> 20)) + rnd;
    /* |x| < 2^-6 (e4m3 subnormals m * 2^-9): x * 2^9 rounded to an integer, nearest even,
     * by the 2^23 magic add; a result of 8 is the least normal, code 0x08 */
    const uint32_t sub = __float_as_uint(__uint_as_float(a) * 512.0f + 8388608.0f) - 0x4B000000u;
    uint32_t r = a < 0x3C800000u ? sub : nrm;
    r = a >= 0x43E00000u ? 0x7Eu : r;
    r = r > 0x7Eu ? 0x7Eu : r;
    r = a > 0x7F800000u ? 0x7Fu : r;
    return s | r;
}

/* Each thread converts 8 consecutive elements (one 16-byte load) and four lanes share a
 * 32-element block; a thread handles up to kQU such chunks of its row, 256 chunks apart,
 * with every load issued before the first conversion so each wave keeps kQU x 1 KB in
 * flight.  K % 32 == 0 keeps every 4-lane group inside the row. */
constexpr int kQU = 4;

__device__ __forceinline__ void r3d_quant_mx8_chunk(r3d_i32x4 raw, uint8_t* q, uint8_t* sx,
                                                    bool write_scale) {
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
    float cv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float c = v[i] * inv;
        if (c > 448.0f) c = 448.0f;
        if (c < -448.0f) c = -448.0f;
        cv[i] = c;
    }
    const uint32_t lo = r3d_e4m3x4_rne(cv[0], cv[1], cv[2], cv[3]);
    const uint32_t hi = r3d_e4m3x4_rne(cv[4], cv[5], cv[6], cv[7]);
    *reinterpret_cast<uint2*>(q) = make_uint2(lo, hi);
    if (write_scale) *sx = (uint8_t)(e + 127);
}

/* UA: the bf16 plane at any element alignment (base or pitch off 16 bytes), each chunk
 * read element by element. */
template <bool UA>
__global__ __launch_bounds__(256) void quant_mx8_kernel(
    const uint16_t* __restrict__ X, int64_t x_pitch, uint8_t* __restrict__ Q, int64_t q_pitch,
    uint8_t* __restrict__ SX, int64_t sx_pitch, int64_t M, int K) {
    /* one workgroup per row; chunk c = 8 elements, 16 bytes */
    const int64_t m = blockIdx.x;
    const int per_row = K >> 3;
    const uint16_t* xr = X + m * x_pitch;
    uint8_t* qr = Q + m * q_pitch;
    uint8_t* sr = SX + m * sx_pitch;
    for (int c0 = threadIdx.x; c0 < per_row; c0 += 256 * kQU) {
        r3d_i32x4 raw[kQU];
#pragma unroll
        for (int u = 0; u < kQU; ++u)
            if (c0 + 256 * u < per_row) {
                const uint16_t* p = xr + 8 * (c0 + 256 * u);
                if (UA) {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        raw[u][j] = (int)((uint32_t)p[2 * j] | ((uint32_t)p[2 * j + 1] << 16));
                } else {
                    raw[u] = *reinterpret_cast<const r3d_i32x4*>(p);
                }
            }
#pragma unroll
        for (int u = 0; u < kQU; ++u) {
            const int c = c0 + 256 * u;
            if (c >= per_row) break;                     /* whole 4-lane groups leave together */
            r3d_quant_mx8_chunk(raw[u], qr + 8 * c, sr + (c >> 2), (threadIdx.x & 3) == 0);
        }
    }
}

}  // namespace r3d

#endif /* R3D_PREFILL_H */
