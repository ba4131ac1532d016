/* r3d_gemv_quad.h -- gfx950 decode GEMV for M <= 4 (gemm_nt_q at mxfp4a8 and fp8a8).
 *
 * At decode the weight planes are the only bytes that matter, so this kernel streams them:
 * every wave fetches its weights D K-steps ahead into a register ring, in whole 128-byte
 * lines straight into the MFMA operand registers, and nothing else rides the vector-memory
 * queue while it runs.  Everything small -- the activation rows and their a_scales (a few
 * KB, read by every workgroup) and the wave's weight scales -- is staged in LDS once, by
 * direct global->LDS loads issued before the ring is primed.
 *
 * Work split: one wave owns a quad (4 consecutive weight rows) and one contiguous chunk of
 * the 128-wide K groups; a workgroup is WV (4 or 8) waves = (WV / chunks) quads x chunks --
 * eight halve the staging bytes per weight row -- so every
 * chunk of a quad sits in the same workgroup and the partials fold through LDS in a fixed
 * order (deterministic).
 *
 * One MFMA step covers 4 consecutive K groups of the quad.  v_mfma_scale_f32_16x16x128
 * sees 16 "rows" in source A; here A row i is (weight row i % 4, group slot i / 4) and
 * source B column j is (group slot j / 4, activation row j % 4).  D[i][j] is the
 * group-partial dot of one weight row with one activation row whenever the two slots agree
 * -- exactly libref's per-group sub (src/r3d_gemm_mxfp4.hip:14-15,
 * src/r3d_gemm_fp8a8.hip:9-15); the other 12 of each 16 products are never read.  In the
 * result layout (lane l holds D[4(l/16) + i][l % 16]) the used values are the 16 lanes
 * l = 20 g + t: slot g, activation row t, weight rows i = 0..3 in the four elements, so the
 * per-group a_scale (and fp8a8 weight scale) multiply whole registers.  Per K step the
 * wave reads 4 rows x 4 groups of weights:
 *   mxfp4a8 : 4 x 256 contiguous bytes in ONE buffer_load_dwordx4 (lane l: row l % 4, group
 *             slot (l / 4) % 4, 32-block l / 16 -- the fp4 operand's own layout); the E8M0
 *             weight scales ride the MFMA's scale operand (exact powers of two);
 *   fp8a8   : 4 x 512 contiguous bytes in TWO loads, the first covering rows 0-1 and the
 *             second rows 2-3 in whole lines; each lane then has one of its two fp8 halves
 *             and its quad neighbour l ^ 2 the other, swapped back with one DPP quad_perm.
 * The B operand (bytes [16kq, +16) and [64 + 16kq, +16) of the lane's group of its
 * activation row) and the used lanes' a_scale and weight scales are read from LDS.
 *
 * Every load is in bounds: rows past N clamp to row N-1, groups past K clamp to the last
 * group, activation rows past M duplicate row M-1; none of these is ever accumulated or
 * stored.  The launch picks a ring depth D no larger than any wave's step count; a wave
 * issues at most D - 1 loads past its chunk, answered as out-of-range (no memory access).
 *
 * LDS: [MT][K + 16] activation bytes (rounded up to 1 KB) at 0, [MT][groups] f32 a_scales
 * at xs_off, then the weight scales at sc_off -- mxfp4a8: the workgroup's rows, whole K,
 * [rows][groups dwords] of E8M0 bytes (sc_bytes in all); fp8a8: sc_bytes per wave of
 * [gmax groups][RB rows] 4-byte slots, bf16 in the low half.
 * The fold reuses the first 1 KB after the K loop. */
#ifndef R3D_GEMV_QUAD_H
#define R3D_GEMV_QUAD_H

#include "r3d_band.h"
#include "r3d_device.h"
#include "r3d_plan.h"

namespace r3d {

/* One K step of one wave in the ring. */
template <int ENC>
struct QuadStep {
    r3d_i32x4 w0;           /* weights (fp8a8: the rows 0-1 load) */
    r3d_i32x4 w1;           /* fp8a8: the rows 2-3 load */
};

/* The weight loads of the step whose group base (for this lane) is `grp` -- or, when `in` is
 * false (a step past the wave's chunk), loads at offsets past the resource's range, which
 * the hardware answers with zeros and no memory access.  Issuing a load either way keeps
 * the code free of conditional loads (whose register merges would cost a full wait in the
 * loop); the two skipped offsets differ so the compiler cannot merge the two loads. */
template <int ENC>
__device__ __forceinline__ QuadStep<ENC> r3d_quad_load(__amdgpu_buffer_rsrc_t r, uint32_t o0,
                                                      uint32_t o1, uint32_t grp, bool in) {
    const uint32_t kSkip = 0x80000000u;
    QuadStep<ENC> v;
    if (ENC == ENC_MXFP4A8) {
        v.w0 = r3d_buf_ld16_stream(r, in ? o0 + 64 * grp : kSkip);
        v.w1 = v.w0;
    } else {
        v.w0 = r3d_buf_ld16_stream(r, in ? o0 + 128 * grp : kSkip);
        v.w1 = r3d_buf_ld16_stream(r, in ? o1 + 128 * grp : kSkip + 64);
    }
    return v;
}

/* Direct global -> LDS load of `BYTES` (16, 4 or 2) per lane, lane l's data landing at LDS
 * byte address lds + l * max(BYTES, 4), issued as inline asm.  The compiler's own LDS-DMA
 * builtin makes it treat every later wait as "all outstanding loads", which would drain the
 * weight ring at every loop iteration; these loads are invisible to it instead.  They are
 * issued before the ring, so any wait the compiler derives for a ring load also covers
 * them (loads retire in order), and the prologue's explicit vmcnt wait publishes them. */
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"   /* m0 is reserved; nothing else here uses it */
template <int BYTES>
__device__ __forceinline__ void r3d_quad_dma(const void* g, uint32_t lds) {
    const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds);
    if (BYTES == 16)
        asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" :: "v"(g), "s"(m0v)
                     : "memory", "m0");
    else if (BYTES == 4)
        asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" :: "v"(g), "s"(m0v)
                     : "memory", "m0");
    else
        asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_ushort %0, off" :: "v"(g), "s"(m0v)
                     : "memory", "m0");
}
#pragma clang diagnostic pop

/* The small launch parameters packed into one argument: M (1..4) in bits 0-2, log2 of the
 * chunk count (0..2) in bits 3-4, fp8a8 weight scales on the 128 x 128 block grid in bit 5,
 * mxfp4a8 scale rows contiguous and 16-byte aligned (1 KB staging loads) in bit 6, a_scale
 * rows at a pitch of K / 128 floats in bit 7. */
constexpr int quad_pack(int M, int log2_chunks, bool rblk128, bool sc16, bool as_dense) {
    return M | (log2_chunks << 3) | ((int)rblk128 << 5) | ((int)sc16 << 6) | ((int)as_dense << 7);
}

/* The arguments every wave needs before its first load come first: the hardware preloads
 * the leading 14 dwords of the argument block into registers at dispatch (the build asks
 * for kernel-argument preloading), so the staging and the ring start without waiting on an
 * argument fetch; as_pitch (M > 1 only), Y and its pitch are fetched as usual.  Pitches in
 * bytes (b, a), bf16 / E8M0 elements (bs) or floats (as), all below 2^31 (quad_fits). */
template <int ENC, int MT, int QPW, int D, int XQ = 0, int WV = 4>
__global__ __launch_bounds__(64 * WV) void gemv_quad_kernel(
    const uint8_t* B, const void* BSv, const uint8_t* A, const float* AS,
    int N, int K, int b_pitch, int bs_pitch, int a_pitch, int pk,
    int as_pitch, uint16_t* __restrict__ Y, int64_t y_pitch) {
    constexpr int LPS = QPW * (ENC == ENC_MXFP4A8 ? 1 : 2);  /* weight loads per step */
    constexpr int RB = 4 * QPW;                               /* weight rows per wave */
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

    const int M = pk & 7;
    const int cl = (pk >> 3) & 3, chunks = 1 << cl;
    const bool rblk128 = (pk >> 5) & 1;
    const bool sc16 = (pk >> 6) & 1;
    const bool as_dense = (pk >> 7) & 1;
    const QuadLds ql = quad_lds(ENC, MT, QPW, WV, K, chunks);
    const int xs_off = (int)ql.xs_off, sc_off = (int)ql.sc_off, sc_bytes = (int)ql.sc_bytes;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int groups = K >> 7;
    const int bpb = WV >> cl;                             /* row blocks per workgroup */
    const int bi = wave >> cl, c = wave & (chunks - 1);
    const int64_t n0 = ((int64_t)blockIdx.x * bpb + bi) * RB;
    const int g0 = (groups * c) >> cl;                    /* groups < 2^21: no overflow */
    const int gc = ((groups * (c + 1)) >> cl) - g0;       /* >= 1: chunks <= groups */
    const int ns = (gc + 3) >> 2;                                     /* K steps of this wave */
    __builtin_assume(ns >= 1);

    const int wr = lane & 3;           /* weight row in the quad (src A) / activation row (src B) */
    const int wg = (lane >> 2) & 3;    /* group slot of this lane's A row and B column */
    const int kq = lane >> 4;          /* 32-wide K block inside the group; slot of used lanes */
    const uint32_t lds0 = (uint32_t)(uintptr_t)smem;      /* LDS byte address of the blob */
    /* weight scales in LDS: mxfp4a8 -- the workgroup's rows, whole K ([rows][groups dwords],
     * the plane's own layout); fp8a8 -- per wave, its chunk ([gmax][RB] 4-byte slots) */
    const int rbw = RB * bpb;                             /* weight rows of the workgroup */
    const uint32_t scl = lds0 + (uint32_t)(sc_off + (ENC == ENC_MXFP4A8 ? 0 : wave * sc_bytes));

    /* ---- 1. LDS staging.  Weight scales first ... */
    if (ENC == ENC_MXFP4A8) {
        const uint8_t* BS8 = reinterpret_cast<const uint8_t*>(BSv);
        const int64_t wn0 = (int64_t)blockIdx.x * rbw;
        if (sc16 && wn0 + rbw <= N) {
            /* the workgroup's rows are one contiguous, 16-byte aligned run of the plane:
             * 1 KB per load (lanes past the run reload its last 16 bytes into padding) */
            const int blk = rbw * 4 * groups;
            for (int i = wave; i < (sc_bytes >> 10); i += WV) {
                const int o = 1024 * i + 16 * lane < blk - 16 ? 1024 * i + 16 * lane : blk - 16;
                r3d_quad_dma<16>(BS8 + wn0 * bs_pitch + o, scl + 1024 * i);
            }
        } else {
            const int nd = rbw * groups;                  /* dwords */
            for (int h = wave; h < (sc_bytes >> 8); h += WV) {
                int e = lane + 64 * h;
                if (e > nd - 1) e = nd - 1;
                const int r = e / groups, d = e - r * groups;
                const int64_t nr = wn0 + r < N ? wn0 + r : N - 1;
                r3d_quad_dma<4>(BS8 + nr * bs_pitch + 4 * (int64_t)d, scl + 256 * h);
            }
        }
    } else {
        const uint16_t* BS16 = reinterpret_cast<const uint16_t*>(BSv);
        for (int h = 0; h < (sc_bytes >> 8); ++h) {
            const int e = lane + 64 * h;
            int d = e / RB;
            if (d > gc - 1) d = gc - 1;
            const int64_t nr = n0 + (e % RB) < N ? n0 + (e % RB) : N - 1;
            const int64_t sr = rblk128 ? nr >> 7 : nr;
            r3d_quad_dma<2>(BS16 + sr * bs_pitch + g0 + d, scl + 256 * h);
        }
    }
    /* ... then the workgroup's activation rows ([MT][K + 16] bytes, whole K) and a_scales
     * ([MT][groups] f32), shared by its WV waves (XQ: quantised here, below) */
    if (!XQ) {
        const int xp = K + 16;
        const int nx = (MT * xp + 1023) >> 10;
        for (int i = wave; i < nx; i += WV) {
            const int b = 1024 * i + 16 * lane;
            int t = 0;                                     /* b / xp, by compares */
#pragma unroll
            for (int j = 1; j <= MT; ++j) t += b >= j * xp;
            int k = b - t * xp;
            if (t > MT - 1) { t = MT - 1; k = K - 16; }
            if (k > K - 16) k = K - 16;
            const int tm = MT == 1 || t < M ? t : M - 1;
            r3d_quad_dma<16>(A + (int64_t)tm * a_pitch + k, lds0 + 1024 * i);
        }
        const int nxs = (MT * groups + 63) >> 6;
        auto stage_as = [&](int64_t asp) {
            for (int h = wave; h < nxs; h += WV) {
                const int e = lane + 64 * h;
                int t = 0;                                 /* e / groups, by compares */
#pragma unroll
                for (int j = 1; j <= MT; ++j) t += e >= j * groups;
                int g = e - t * groups;
                if (t > MT - 1) { t = MT - 1; g = groups - 1; }
                const int tm = MT == 1 || t < M ? t : M - 1;
                r3d_quad_dma<4>(AS + (int64_t)tm * asp + g, lds0 + xs_off + 256 * h);
            }
        };
        /* one row, or rows at a pitch of groups floats: as_pitch (an argument past the
         * preloaded ones, fetched on the other branch only) does not enter the address */
        if (MT == 1 || as_dense) stage_as(groups);
        else stage_as(as_pitch);
    }

    /* ---- 2. the weight stream, through a buffer resource over the wave's RB rows */
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(B + n0 * b_pitch), (short)0, (int)(RB * b_pitch), 0x00020000);
    uint32_t wo0[QPW], wo1[QPW];
#pragma unroll
    for (int q = 0; q < QPW; ++q) {
        const int64_t rq = n0 + 4 * q;
        if (ENC == ENC_MXFP4A8) {
            const int64_t nr = rq + wr < N ? rq + wr : N - 1;
            wo0[q] = (uint32_t)((nr - n0) * b_pitch + 16 * kq);
            wo1[q] = wo0[q];
        } else {
            /* load 0 covers rows 0-1 of the quad, load 1 rows 2-3, each in whole 128-byte
             * groups: a lane fetches its own low half (bytes [16kq, +16) of the group) from
             * the pair that holds its row and the high half ([64 + 16kq, +16)) of lane
             * l ^ 2's row from the other */
            const int64_t r0 = rq + (wr & 1) < N ? rq + (wr & 1) : N - 1;
            const int64_t r1 = rq + 2 + (wr & 1) < N ? rq + 2 + (wr & 1) : N - 1;
            wo0[q] = (uint32_t)((r0 - n0) * b_pitch + 16 * kq + (wr >= 2 ? 64 : 0));
            wo1[q] = (uint32_t)((r1 - n0) * b_pitch + 16 * kq + (wr < 2 ? 64 : 0));
        }
    }
    auto grp_of = [&](int s) -> uint32_t {
        const int g = g0 + 4 * s + wg;
        return (uint32_t)(g < groups ? g : groups - 1);
    };

    struct Step { QuadStep<ENC> q[QPW]; };
    auto load = [&](int s) {
        Step v;
#pragma unroll
        for (int q = 0; q < QPW; ++q)
            v.q[q] = r3d_quad_load<ENC>(wrs, wo0[q], wo1[q], grp_of(s), s < ns);
        return v;
    };

    /* XQ: the activations arrive as bf16 rows (A, a_pitch bytes) and are quantised into the
     * same LDS images with quant_act_fp8's arithmetic over groups of 128 (src/r3d_band.hip:
     * 117-153): amax = max |x| (NaN never wins), sc = amax > 0 ? amax / 448 : 1 (as
     * amax * (1/448)), q = e4m3_rne(clamp(x * (1 / sc), +-448)) -- the codes and scales the
     * quant_act_fp8 row writes, so the products are those of the unfused pair.  A lane takes
     * one 16-byte chunk (8 values) of the [MT][K / 8] chunk space per block of 64 chunks; a
     * group is 16 consecutive chunks, i.e. 16 lanes, reduced by 4 xor-shuffles (a row's
     * K / 8 chunks are whole groups, so no group straddles two rows).  Wave w takes blocks
     * w, w + WV, ...; XU blocks per batch, the first batch's loads issued before the weight
     * ring is primed (so waiting for them never waits for weights).  One batch covers
     * MT * K <= 2048 * WV; more takes further batches, whose loads wait behind the ring's.
     * Every workgroup re-reads the bf16 rows (twice the bytes of the e4m3 images) and
     * re-quantises them: at MT = 4 that costs more than the producer launch it saves at the
     * benchmark shapes, so the plan takes MT = 4 only when the engine asks (tunable "fuse"). */
    constexpr int XU = XQ ? 4 : 1;
    const int cpr = K >> 3, nchunk = MT * cpr;
    const int nxb = (nchunk + 63) >> 6;
    r3d_i32x4 xv[XU];
    auto xq_load = [&](int batch) {
#pragma unroll
        for (int u = 0; u < XU; ++u) {
            const int c0 = 64 * (wave + WV * (batch * XU + u)) + lane;
            const int c = c0 < nchunk ? c0 : nchunk - 1;
            int t = 0;                                     /* c / cpr, by compares */
#pragma unroll
            for (int j = 1; j < MT; ++j) t += c >= j * cpr;
            const int k = 8 * (c - t * cpr);
            const int tm = MT == 1 || t < M ? t : M - 1;
            xv[u] = *reinterpret_cast<const r3d_i32x4*>(A + (int64_t)tm * a_pitch + 2 * k);
        }
    };
    auto xq_store = [&](int batch) {
        float* xst = reinterpret_cast<float*>(smem + xs_off);
#pragma unroll
        for (int u = 0; u < XU; ++u) {
            const int c = 64 * (wave + WV * (batch * XU + u)) + lane;
            float v[8];
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[2 * i] = __uint_as_float((uint32_t)xv[u][i] << 16);
                v[2 * i + 1] = __uint_as_float((uint32_t)xv[u][i] & 0xFFFF0000u);
                amax = fmaxf(amax, fmaxf(fabsf(v[2 * i]), fabsf(v[2 * i + 1])));
            }
#pragma unroll
            for (int off = 8; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
            if (c < nchunk) {                              /* whole 16-lane groups */
                int t = 0;
#pragma unroll
                for (int j = 1; j < MT; ++j) t += c >= j * cpr;
                const int k = 8 * (c - t * cpr);
                const float sc = amax > 0.0f ? amax * (1.0f / 448.0f) : 1.0f;
                const float inv = 1.0f / sc;
                float cv[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) cv[i] = r3d_band_clamp448(v[i] * inv);
                *reinterpret_cast<uint2*>(smem + t * (K + 16) + k) =
                    make_uint2(r3d_e4m3x4_rne(cv[0], cv[1], cv[2], cv[3]),
                               r3d_e4m3x4_rne(cv[4], cv[5], cv[6], cv[7]));
                if ((lane & 15) == 0) xst[t * groups + (k >> 7)] = sc;
            }
        }
    };
    if (XQ) xq_load(0);
    __builtin_amdgcn_sched_barrier(0);

    /* Scheduling barriers keep each step's loads in step order, in the prologue as in the
     * loop, so every wait is "the oldest step's loads".  The launch picks D <= ns. */
    Step ring[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        ring[d] = load(d);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (XQ) {
        for (int b = 0;;) {
            xq_store(b);
            if (++b * WV * XU >= nxb) break;
            xq_load(b);
        }
        /* the quantised rows are this wave's LDS writes: publish them with the staging */
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" :: "n"(D * LPS) : "memory");
    } else {
        /* this wave's LDS loads are all but the newest D*LPS loads in flight: wait for
         * them, then meet the other waves */
        asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" :: "n"(D * LPS) : "memory");
    }

    /* ---- 3. consume: B operand, a_scale and weight scales from LDS.  These are ordinary
     * LDS reads: the compiler knows nothing of the LDS fill (inline asm above), so it
     * waits only on lgkmcnt for them. */
    const int tB = MT == 1 ? 0 : wr;
    const uint8_t* xrow = smem + tB * (K + 16) + 16 * kq;
    const float* xs = reinterpret_cast<const float*>(smem + xs_off) + tB * groups;
    const uint8_t* sc = smem + sc_off + (ENC == ENC_MXFP4A8 ? 0 : wave * sc_bytes);
    r3d_f32x4 acc[QPW];
#pragma unroll
    for (int q = 0; q < QPW; ++q) acc[q] = r3d_f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    auto consume = [&](const Step& v, int s) {
        const uint32_t gb = grp_of(s);
        const r3d_i32x4 lo = *reinterpret_cast<const r3d_i32x4*>(xrow + 128 * gb);
        const r3d_i32x4 hi = *reinterpret_cast<const r3d_i32x4*>(xrow + 128 * gb + 64);
        const r3d_i32x8 bv = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        const int su = 4 * s + kq;                        /* the used lanes' slot in the chunk */
        const float a_s = xs[g0 + su < groups ? g0 + su : groups - 1];
        const bool live = su < gc;
#pragma unroll
        for (int q = 0; q < QPW; ++q) {
            if (ENC == ENC_MXFP4A8) {
                const int sl = 4 * s + wg < gc ? 4 * s + wg : gc - 1;
                const int sa = sc[(bi * RB + 4 * q + wr) * 4 * groups + 4 * (g0 + sl) + kq];
                const r3d_f32x4 d = r3d_mfma_fp4_fp8(v.q[q].w0, sa, bv, R3D_E8M0_ONE);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[q][i] += live ? d[i] * a_s : 0.0f;
            } else {
                const bool own = wr < 2;
                r3d_i32x4 wl, wh;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    wl[i] = own ? v.q[q].w0[i] : v.q[q].w1[i];
                    /* quad_perm [2,3,0,1]: lane l takes lane l ^ 2's other half */
                    wh[i] = __builtin_amdgcn_mov_dpp(own ? v.q[q].w1[i] : v.q[q].w0[i], 0x4E,
                                                     0xF, 0xF, false);
                }
                const r3d_i32x8 wv = {wl[0], wl[1], wl[2], wl[3], wh[0], wh[1], wh[2], wh[3]};
                const r3d_f32x4 d = r3d_mfma_fp8_fp8(wv, bv);
                const int sl = su < gc ? su : gc - 1;
                const r3d_i32x4 sb = *reinterpret_cast<const r3d_i32x4*>(sc + 4 * (sl * RB + 4 * q));
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float sbv = __uint_as_float((uint32_t)sb[i] << 16);
                    acc[q][i] += live ? (d[i] * a_s) * sbv : 0.0f;
                }
            }
        }
    };

    /* Whole blocks of D steps while a full block of real loads remains; then one block that
     * loads the last (fewer than D) steps, skipping the rest; then the last steps, with no
     * loads.  Every wave loads and consumes exactly its ns steps (plus at most D - 1
     * skipped loads). */
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

    /* The accumulators are complete here in every lane: without this the compiler may sink
     * the last MFMAs into the used-lanes-only branch below, where a partial exec mask
     * corrupts them (an MFMA reads its operands across the whole wave). */
#pragma unroll
    for (int q = 0; q < QPW; ++q) asm volatile("" : "+v"(acc[q]));

    /* ---- 4. fold: used lanes (kq == wg) hold slot kq's partials of activation row wr;
     * sum slots then chunks in a fixed order */
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");   /* LDS reads done */
    r3d_f32x4* red = reinterpret_cast<r3d_f32x4*>(smem);
    if (kq == wg)
#pragma unroll
        for (int q = 0; q < QPW; ++q) red[(wave * QPW + q) * 16 + 4 * kq + wr] = acc[q];
    __syncthreads();
    const int tid = threadIdx.x;
    if (tid < bpb * RB * MT) {
        const int b = tid / (RB * MT), r = (tid / MT) % RB, t = tid % MT;
        const int q = r >> 2, i = r & 3;
        const float* rf = reinterpret_cast<const float*>(smem);
        float y = 0.0f;
        for (int cc = 0; cc < chunks; ++cc)
            for (int g = 0; g < 4; ++g)
                y += rf[(((b * chunks + cc) * QPW + q) * 16 + 4 * g + t) * 4 + i];
        const int64_t n = ((int64_t)blockIdx.x * bpb + b) * RB + r;
        if (t < M && n < N) Y[(int64_t)t * y_pitch + n] = r3d_bf16_rne(y);
    }
}

}  // namespace r3d

#endif /* R3D_GEMV_QUAD_H */
