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
 * the 128-wide K groups; a workgroup is 4 waves = (4 / chunks) quads x chunks, so every
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
 * stored.  Each wave loads exactly its chunk's steps: the launch picks a ring depth D no
 * larger than any wave's step count, and the last steps run as a static tail.
 *
 * LDS: [MT][K + 16] activation bytes (rounded up to 1 KB) at 0, [MT][groups] f32 a_scales
 * at xs_off, then per wave sc_bytes of weight scales at sc_off -- mxfp4a8: [4 rows][gmax
 * dwords] of E8M0 bytes, fp8a8: [gmax groups][4 rows] 4-byte slots, bf16 in the low half.
 * The fold reuses the first 1 KB after the K loop. */
#ifndef R3D_GEMV_QUAD_H
#define R3D_GEMV_QUAD_H

#include "r3d_device.h"
#include "r3d_plan.h"

namespace r3d {

/* One K step of one wave in the ring. */
template <int ENC>
struct QuadStep {
    r3d_i32x4 w0;           /* weights (fp8a8: the rows 0-1 load) */
    r3d_i32x4 w1;           /* fp8a8: the rows 2-3 load */
};

/* The weight loads of the step whose group base (for this lane) is `grp`. */
template <int ENC>
__device__ __forceinline__ QuadStep<ENC> r3d_quad_load(__amdgpu_buffer_rsrc_t r, uint32_t o0,
                                                      uint32_t o1, uint32_t grp) {
    QuadStep<ENC> v;
    if (ENC == ENC_MXFP4A8) {
        v.w0 = r3d_buf_ld16_stream(r, o0 + 64 * grp);
        v.w1 = v.w0;
    } else {
        v.w0 = r3d_buf_ld16_stream(r, o0 + 128 * grp);
        v.w1 = r3d_buf_ld16_stream(r, o1 + 128 * grp);
    }
    return v;
}

/* The last 2D - 1 or fewer steps of the ring walk, T of them still to load: consume the D
 * ring slots, refilling the first T, then consume those T.  T is a compile-time constant
 * so every slot index and load is static (no conditional load, hence no register merge
 * and no full wait in the compiled code).  quad_tail_at picks T at run time. */
template <int T, int D, typename Ring, typename Consume, typename Load>
__device__ __forceinline__ void quad_tail(Ring& ring, int s0, Consume& consume, Load& load) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
        consume(ring[d], s0 + d);
        if (d < T) ring[d] = load(s0 + d + D);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int d = 0; d < T; ++d) {
        consume(ring[d], s0 + D + d);
        __builtin_amdgcn_sched_barrier(0);
    }
}

template <int T, int D, typename Ring, typename Consume, typename Load>
__device__ __forceinline__ void quad_tail_at(int t, Ring& ring, int s0, Consume& consume,
                                             Load& load) {
    if (t == T) {
        quad_tail<T, D>(ring, s0, consume, load);
    } else if constexpr (T + 1 < D) {
        quad_tail_at<T + 1, D>(t, ring, s0, consume, load);
    }
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

/* One step's LDS operands -- the B fragment (two 16-byte reads), the used lanes' a_scale,
 * and the weight scale(s) -- read in one asm block that also waits for them.  The compiler
 * cannot see these reads, which is the point: LDS filled by direct global->LDS loads would
 * otherwise make it wait for every outstanding global load (the whole weight ring) before
 * each step.  The fill is complete and published by the s_waitcnt + s_barrier that ends
 * the prologue. */
struct QuadLds {
    r3d_i32x4 lo, hi;
    float as;
    r3d_i32x4 sb;           /* fp8a8: 4 slots of bf16 weight scales; mxfp4a8: sb[0] = E8M0 */
};

template <int ENC>
__device__ __forceinline__ QuadLds r3d_quad_lds(uint32_t x, uint32_t a, uint32_t sc) {
    QuadLds r;
    if (ENC == ENC_MXFP4A8) {
        int e;
        asm volatile(
            "ds_read_b128 %0, %4\n\t"
            "ds_read_b128 %1, %4 offset:64\n\t"
            "ds_read_b32 %2, %5\n\t"
            "ds_read_u8 %3, %6\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(r.lo), "=&v"(r.hi), "=&v"(r.as), "=&v"(e)
            : "v"(x), "v"(a), "v"(sc));
        r.sb = r3d_i32x4{e, 0, 0, 0};
    } else {
        asm volatile(
            "ds_read_b128 %0, %4\n\t"
            "ds_read_b128 %1, %4 offset:64\n\t"
            "ds_read_b32 %2, %5\n\t"
            "ds_read_b128 %3, %6\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(r.lo), "=&v"(r.hi), "=&v"(r.as), "=&v"(r.sb)
            : "v"(x), "v"(a), "v"(sc));
    }
    return r;
}

template <int ENC, int MT, int D>
__global__ __launch_bounds__(256) void gemv_quad_kernel(
    const uint8_t* A, const float* AS, const uint8_t* B, const void* BSv,
    uint16_t* __restrict__ Y,
    int M, int N, int K, int chunks, int rblk, int gmax, int xs_off, int sc_off, int sc_bytes,
    int64_t a_pitch, int64_t as_pitch, int64_t b_pitch, int64_t bs_pitch, int64_t y_pitch) {
    constexpr int LPS = ENC == ENC_MXFP4A8 ? 1 : 2;        /* weight loads per step */
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int groups = K >> 7;
    const int qpb = 4 / chunks;                           /* quads per workgroup */
    const int qi = wave / chunks, c = wave % chunks;
    const int64_t n0 = ((int64_t)blockIdx.x * qpb + qi) * 4;
    const int g0 = (int)((int64_t)groups * c / chunks);
    const int gc = (int)((int64_t)groups * (c + 1) / chunks) - g0;   /* >= 1: chunks <= groups */
    const int ns = (gc + 3) >> 2;                                     /* K steps of this wave */
    __builtin_assume(ns >= 1);

    const int wr = lane & 3;           /* weight row in the quad (src A) / activation row (src B) */
    const int wg = (lane >> 2) & 3;    /* group slot of this lane's A row and B column */
    const int kq = lane >> 4;          /* 32-wide K block inside the group; slot of used lanes */
    const uint32_t lds0 = (uint32_t)(uintptr_t)smem;      /* LDS byte address of the blob */
    const uint32_t scl = lds0 + (uint32_t)(sc_off + wave * sc_bytes);   /* this wave's scales */

    /* ---- 1. LDS staging.  The wave's weight scales first ... */
    {
        const uint8_t* BS8 = reinterpret_cast<const uint8_t*>(BSv);
        const uint16_t* BS16 = reinterpret_cast<const uint16_t*>(BSv);
        for (int h = 0; h < (sc_bytes >> 8); ++h) {
            const int e = lane + 64 * h;
            if (ENC == ENC_MXFP4A8) {
                int r = e / gmax, d = e - r * gmax;
                if (r > 3) r = 3;
                if (d > gc - 1) d = gc - 1;
                const int64_t nr = n0 + r < N ? n0 + r : N - 1;
                r3d_quad_dma<4>(BS8 + nr * bs_pitch + 4 * (int64_t)(g0 + d), scl + 256 * h);
            } else {
                int d = e >> 2;
                if (d > gc - 1) d = gc - 1;
                const int64_t nr = n0 + (e & 3) < N ? n0 + (e & 3) : N - 1;
                const int64_t sr = rblk == 1 ? nr : nr >> 7;
                r3d_quad_dma<2>(BS16 + sr * bs_pitch + g0 + d, scl + 256 * h);
            }
        }
    }
    /* ... then the workgroup's activation rows ([MT][K + 16] bytes, whole K) and a_scales
     * ([MT][groups] f32), shared by its 4 waves */
    {
        const int xp = K + 16;
        const int nx = (MT * xp + 1023) >> 10;
        for (int i = wave; i < nx; i += 4) {
            const int b = 1024 * i + 16 * lane;
            int t = b / xp, k = b - t * xp;
            if (t > MT - 1) { t = MT - 1; k = K - 16; }
            if (k > K - 16) k = K - 16;
            const int tm = t < M ? t : M - 1;
            r3d_quad_dma<16>(A + (int64_t)tm * a_pitch + k, lds0 + 1024 * i);
        }
        const int nxs = (MT * groups + 63) >> 6;
        for (int h = wave; h < nxs; h += 4) {
            const int e = lane + 64 * h;
            int t = e / groups, g = e - t * groups;
            if (t > MT - 1) { t = MT - 1; g = groups - 1; }
            const int tm = t < M ? t : M - 1;
            r3d_quad_dma<4>(AS + (int64_t)tm * as_pitch + g, lds0 + xs_off + 256 * h);
        }
    }

    /* ---- 2. the weight stream, through a buffer resource over the quad's 4 rows */
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(B + n0 * b_pitch), (short)0, (int)(4 * b_pitch), 0x00020000);
    uint32_t wo0, wo1;
    if (ENC == ENC_MXFP4A8) {
        const int64_t nr = n0 + wr < N ? n0 + wr : N - 1;
        wo0 = (uint32_t)((nr - n0) * b_pitch + 16 * kq);
        wo1 = wo0;
    } else {
        /* load 0 covers rows 0-1, load 1 rows 2-3, each in whole 128-byte groups: a lane
         * fetches its own low half (bytes [16kq, +16) of the group) from the pair that holds
         * its row and the high half ([64 + 16kq, +16)) of lane l ^ 2's row from the other */
        const int64_t r0 = n0 + (wr & 1) < N ? n0 + (wr & 1) : N - 1;
        const int64_t r1 = n0 + 2 + (wr & 1) < N ? n0 + 2 + (wr & 1) : N - 1;
        wo0 = (uint32_t)((r0 - n0) * b_pitch + 16 * kq + (wr >= 2 ? 64 : 0));
        wo1 = (uint32_t)((r1 - n0) * b_pitch + 16 * kq + (wr < 2 ? 64 : 0));
    }
    auto grp_of = [&](int s) -> uint32_t {
        const int g = g0 + 4 * s + wg;
        return (uint32_t)(g < groups ? g : groups - 1);
    };

    auto load = [&](int s) { return r3d_quad_load<ENC>(wrs, wo0, wo1, grp_of(s)); };

    /* Scheduling barriers keep each step's loads in step order, in the prologue as in the
     * loop, so every wait is "the oldest step's loads".  The launch picks D <= ns. */
    QuadStep<ENC> ring[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        ring[d] = load(d);
        __builtin_amdgcn_sched_barrier(0);
    }
    /* this wave's LDS loads are all but the newest D*LPS loads in flight: wait for them,
     * then meet the other waves */
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" :: "n"(D * LPS) : "memory");

    /* ---- 3. consume: B operand, a_scale and weight scales from LDS (byte addresses) */
    const int tB = MT == 1 ? 0 : wr;
    const uint32_t xrow = lds0 + (uint32_t)(tB * (K + 16) + 16 * kq);
    const uint32_t xs = lds0 + (uint32_t)(xs_off + 4 * tB * groups);
    r3d_f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};

    auto consume = [&](const QuadStep<ENC>& v, int s) {
        const int su = 4 * s + kq;                        /* the used lanes' slot in the chunk */
        const int gs = g0 + su < groups ? g0 + su : groups - 1;
        uint32_t sca;
        if (ENC == ENC_MXFP4A8) {
            const int sl = 4 * s + wg < gc ? 4 * s + wg : gc - 1;
            sca = scl + (uint32_t)(wr * 4 * gmax + 4 * sl + kq);
        } else {
            sca = scl + (uint32_t)(16 * (su < gc ? su : gc - 1));
        }
        const QuadLds l = r3d_quad_lds<ENC>(xrow + 128 * grp_of(s), xs + 4 * (uint32_t)gs, sca);
        const r3d_i32x8 bv = {l.lo[0], l.lo[1], l.lo[2], l.lo[3], l.hi[0], l.hi[1], l.hi[2], l.hi[3]};
        const bool live = su < gc;
        if (ENC == ENC_MXFP4A8) {
            const r3d_f32x4 d = r3d_mfma_fp4_fp8(v.w0, l.sb[0], bv, R3D_E8M0_ONE);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] += live ? d[i] * l.as : 0.0f;
        } else {
            const bool own = wr < 2;
            r3d_i32x4 wl, wh;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                wl[i] = own ? v.w0[i] : v.w1[i];
                /* quad_perm [2,3,0,1]: lane l takes lane l ^ 2's other half */
                wh[i] = __builtin_amdgcn_mov_dpp(own ? v.w1[i] : v.w0[i], 0x4E, 0xF, 0xF, false);
            }
            const r3d_i32x8 wv = {wl[0], wl[1], wl[2], wl[3], wh[0], wh[1], wh[2], wh[3]};
            const r3d_f32x4 d = r3d_mfma_fp8_fp8(wv, bv);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float sbv = __uint_as_float((uint32_t)l.sb[i] << 16);
                acc[i] += live ? (d[i] * l.as) * sbv : 0.0f;
            }
        }
    };

    /* whole blocks of D steps while a full block of loads remains, then the static tail:
     * exactly ns steps are loaded and consumed */
    int s0 = 0;
    for (; s0 + 2 * D <= ns; s0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            consume(ring[d], s0 + d);
            ring[d] = load(s0 + d + D);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    quad_tail_at<0, D>(ns - s0 - D, ring, s0, consume, load);

    /* ---- 4. fold: used lanes (kq == wg) hold slot kq's partials of activation row wr;
     * sum slots then chunks in a fixed order */
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");   /* LDS reads done */
    r3d_f32x4* red = reinterpret_cast<r3d_f32x4*>(smem);
    if (kq == wg) red[wave * 16 + 4 * kq + wr] = acc;
    __syncthreads();
    const int tid = threadIdx.x;
    if (tid < qpb * 4 * MT) {
        const int q = tid / (4 * MT), i = (tid / MT) & 3, t = tid % MT;
        const float* rf = reinterpret_cast<const float*>(smem);
        float y = 0.0f;
        for (int cc = 0; cc < chunks; ++cc)
            for (int g = 0; g < 4; ++g) y += rf[((q * chunks + cc) * 16 + 4 * g + t) * 4 + i];
        const int64_t n = n0 - 4 * qi + 4 * q + i;
        if (t < M && n < N) Y[(int64_t)t * y_pitch + n] = r3d_bf16_rne(y);
    }
}

}  // namespace r3d

#endif /* R3D_GEMV_QUAD_H */
