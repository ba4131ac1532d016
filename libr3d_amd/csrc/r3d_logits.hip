/* r3d_logits.hip -- the gfx950 logits_gemm_e4m3 row: logits over a joined e4m3 +
 * block-scale lm_head (the reference's row is src/r3d_gemm_logits.hip:72-226; its layout
 * hooks, :233-272, are r3d_head.cpp's).
 *
 *     y[m, n] = sum_k x[m, k] * e4m3(codes[n, k]) * scale[n / br, k / 128]     (f32 out)
 *
 * On MFMA.  A decoded e4m3 code has 4 significant bits and an exponent inside bf16's range,
 * so it is exact in bf16 (v_cvt_scalef32_pk_bf16_fp8 at scale 1 reproduces all 256 codes,
 * NaN included); x is bf16 already.  v_mfma_f32_16x16x32_bf16 therefore forms every product
 * x * code exactly -- 8 x 4 significant bits -- and sums 32 of them at f32 accuracy (worst
 * measured on MI355X: 5.9 * 2^-24 of the sum of magnitudes per instruction, C included).
 * The scale, which need not be a power of two, is applied once per 128-wide block, in f32:
 * tot = fma(scale, block_sum, tot).  This differs from the reference's order (one fma per
 * product, code * scale rounded first) only in where the f32 roundings fall; both stay
 * within (block count + 4 * 66) * 2^-24 * sum |x * code * scale| of the exact sum.
 *
 * The walk (logits_e4m3_kernel below): 16 head rows a chunk, in 256-wide windows; one
 * buffer_load_dwordx4 a lane reads 4 head rows x 256 contiguous bytes ("the quad trick":
 * MFMA A row i = (head row i % 4, K slot i / 4), B column j = (K slot j / 4, activation
 * row j % 4), the products where the slots agree are used); activation rows staged once
 * per workgroup in LDS; each chunk's scales in an LDS table; waves walk chunks
 * blocks * waves apart with a register ring running across chunk boundaries.  n_embd off a
 * multiple of 16, or x, codes or scale off the vector walk's alignment, take the same walk
 * with every piece read by aligned dwords and funnel-shifted (UA). */
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <mutex>
#include <stddef.h>
#include <stdio.h>
#include <string.h>

#include "r3d_device.h"
#include "r3d_dump.h"
#include "r3d_gemm_any.h"
#include "r3d_plan.h"
#include "rad_planes.h"
#include "rad_plugin.h"

namespace r3d {

typedef __bf16 lg_bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 lg_bf16x2 __attribute__((ext_vector_type(2)));

/* Eight e4m3 codes (two dwords, byte 0 first) -> eight bf16, exact. */
__device__ __forceinline__ lg_bf16x8 lg_codes8(int w0, int w1) {
    const lg_bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((unsigned)w0, 1.0f, false);
    const lg_bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((unsigned)w0, 1.0f, true);
    const lg_bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((unsigned)w1, 1.0f, false);
    const lg_bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((unsigned)w1, 1.0f, true);
    return lg_bf16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

/* One scale element (bf16, f16 or f32 by SDT 0/1/2) at byte `off` of the plane, widened
 * exactly; an offset past the plane reads 0. */
template <int SDT>
__device__ __forceinline__ float lg_scale(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
    if (SDT == 2) return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, (int)off, 0, 0));
    const uint32_t v = __builtin_amdgcn_raw_buffer_load_b16(rs, (int)off, 0, 0);
    if (SDT == 0) return __uint_as_float(v << 16);
    return __half2float(__ushort_as_half((unsigned short)v));
}

/* One scale element at any alignment (the dword walk): widened exactly. */
template <int SDT>
__device__ __forceinline__ float lg_scale_any(const AnyBuf& b, uint32_t off) {
    const uint32_t v = any_ld4(b, off);
    if (SDT == 2) return __uint_as_float(v);
    if (SDT == 0) return __uint_as_float(v << 16);
    return __half2float(__ushort_as_half((unsigned short)(v & 0xFFFFu)));
}

/* The device copy of the header still describes the planes the host planned from.  Read
 * by aligned dwords (the blob may start at any byte). */
__device__ __forceinline__ bool lg_header_ok(const LogitsGuard& g) {
    const int ne = (g.ic > g.is ? g.ic : g.is) + 1;
    const uint32_t eb = (uint32_t)sizeof(RadPlanesHeader), es = (uint32_t)sizeof(RadPlanesEntry);
    const AnyBuf hb = any_buf(g.header, eb + es * ne);
    auto u32 = [&](uint32_t o) { return any_ld4(hb, o); };
    auto i64 = [&](uint32_t o) {
        return (int64_t)((uint64_t)any_ld4(hb, o) | ((uint64_t)any_ld4(hb, o + 4) << 32));
    };
    if (u32(offsetof(RadPlanesHeader, magic)) != RAD_PLANES_MAGIC ||
        u32(offsetof(RadPlanesHeader, n_planes)) != 2)
        return false;
    const uint32_t c = eb + es * g.ic, s = eb + es * g.is;
    return u32(c + offsetof(RadPlanesEntry, dtype)) == RAD_F8E4M3 &&
           i64(c + offsetof(RadPlanesEntry, offset)) == g.c_off &&
           i64(c + offsetof(RadPlanesEntry, rows)) == g.c_rows &&
           i64(c + offsetof(RadPlanesEntry, cols)) == g.c_cols &&
           u32(s + offsetof(RadPlanesEntry, dtype)) == g.s_dtype &&
           i64(s + offsetof(RadPlanesEntry, offset)) == g.s_off &&
           i64(s + offsetof(RadPlanesEntry, rows)) == g.s_rows &&
           i64(s + offsetof(RadPlanesEntry, row_bytes)) == g.s_row_bytes &&
           i64(s + offsetof(RadPlanesEntry, block)) == g.s_br;
}

constexpr uint32_t kLgOob = 0x80000000u;     /* past every buffer's num_records: reads 0 */

/* A chunk is 16 head rows (four groups of 4) over the whole of K, walked in 256-wide
 * windows.  v_mfma_f32_16x16x32_bf16 sees 16 "rows" in source A; here A row i is (head row
 * i % 4 of the group, K slot i / 4) and source B column j is (K slot j / 4, activation row
 * j % 4): lane l = 16 kq + 4 slot + lr holds, for head row lr and activation row lr, the
 * 16 bytes [64 slot + 16 kq, +16) of the window -- one buffer_load_dwordx4 per group and
 * window reads the group's 4 rows x 256 contiguous bytes.  Each 8-byte half feeds one MFMA;
 * D[i][j] is a slot-partial dot product whenever the two slots agree, which in the result
 * layout (lane l holds D[4 (l/16) + v][l % 16]) are the lanes l = 20 s + t: slot s,
 * activation row t, head rows v = 0..3 in the four elements (the other 12 of each 16 are
 * never read).  Slots 0-1 lie in the window's first 128-wide scale block, 2-3 in its
 * second, so the chunk's scale table in LDS ([block][16 rows] f32) gives each used lane its
 * four rows' scales with one ds_read_b128.  After the K walk the four slot lanes of each
 * (activation row, head row) are summed in slot order.  Activation rows beyond 4 take
 * further MFMAs on the same A operand (XG groups of 4).
 *
 * Persistent: a workgroup stages its activation rows once, and each wave walks the chunks
 * blocks * waves apart as one stream of windows -- the register ring (D windows in flight)
 * runs straight across chunk boundaries.  The next chunk's scales are loaded into registers
 * when a chunk starts and written over the wave's table when it ends: a full chunk of a
 * per-row scale grid whose 16 rows form one 16-byte aligned span of whole 16-byte units is
 * fetched by the unit (at most kLgTU a lane); a per-128-rows grid's one scale row by the
 * element; anything else by the table value (the first 4 kLgTU a lane ahead, the rest when
 * the chunk ends). */
constexpr int kLgTU = 2;                              /* 16-byte units a lane prefetches */

/* Element i (0..15 / ESZ) of a 16-byte unit of scale elements, widened exactly. */
template <int SDT>
__device__ __forceinline__ float lg_unit_elem(const r3d_i32x4& u, int i) {
    if (SDT == 2) return __int_as_float(u[i]);
    const uint32_t h = (uint32_t)u[i >> 1] >> (16 * (i & 1)) & 0xFFFFu;
    if (SDT == 0) return __uint_as_float(h << 16);
    return __half2float(__ushort_as_half((unsigned short)h));
}

template <int D, int XG, int SDT, bool UA>
__global__ __launch_bounds__(512) void logits_e4m3_kernel(
    const uint16_t* __restrict__ X, int64_t x_pitch, const uint8_t* __restrict__ codes,
    const uint8_t* __restrict__ scale, int64_t s_pitch, int64_t s_bytes, int br,
    float* __restrict__ Y, int64_t y_pitch, int N, int K, int M, int mt, int nwin,
    int nw_pad, int xrow, int xbytes, int64_t chunks, LogitsGuard guard) {
    static_assert(D >= 1 && D <= 3, "one to three windows in flight");
    constexpr int ESZ = SDT == 2 ? 4 : 2;
    constexpr int RS = D + 1;                         /* register ring: one window read, D in flight */
    extern __shared__ __align__(16) uint8_t lg_lds[];
    const int nwaves = blockDim.x >> 6;
    const int mb = blockIdx.y * mt;
    const int live = M - mb < mt ? M - mb : mt;

    /* stage x rows [mb, mb + live) as bf16, zero from K to nw_pad windows of 256; a row is
     * xrow bytes apart (nw_pad * 512 + 16: the 16 keeps the four rows a B-operand read
     * touches on different banks) */
    const int cpr = nw_pad * 32;                      /* 16-byte chunks per staged row */
    for (int i = threadIdx.x; i < live * cpr; i += blockDim.x) {
        const int m = i / cpr, c = i - m * cpr;
        r3d_i32x4 v = {0, 0, 0, 0};
        const uint16_t* xp = X + (int64_t)(mb + m) * x_pitch + 8 * c;
        if (UA) {                                     /* element by element, zero past K */
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t lo = 8 * c + 2 * j < K ? xp[2 * j] : 0u;
                const uint32_t hi = 8 * c + 2 * j + 1 < K ? xp[2 * j + 1] : 0u;
                v[j] = (int)(lo | (hi << 16));
            }
        } else if (8 * c < K) {
            v = *reinterpret_cast<const r3d_i32x4*>(xp);
        }
        *reinterpret_cast<r3d_i32x4*>(lg_lds + m * xrow + 16 * c) = v;
    }
    __syncthreads();

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l = threadIdx.x & 63, kq = l >> 4, slot = (l >> 2) & 3, lr = l & 3;
    const int64_t ch0 = (int64_t)blockIdx.x * nwaves + wave, stride = (int64_t)gridDim.x * nwaves;
    if (ch0 >= chunks) return;
    const int nch = (int)((chunks - ch0 + stride - 1) / stride);
    if (!lg_header_ok(guard)) {                       /* the head changed under the plan */
        for (int k = 0; k < nch; ++k)
            for (int i = l; i < 16 * live; i += 64) {
                const int64_t row = (ch0 + k * stride) * 16 + (i & 15);
                if (row < N) Y[(int64_t)(mb + (i >> 4)) * y_pitch + row] = __builtin_nanf("");
            }
        return;
    }
    const int nb_pad = 2 * nw_pad;                    /* scale blocks in a table */
    float* tab = reinterpret_cast<float*>(lg_lds + xbytes) + (size_t)wave * 16 * nb_pad;
    const __amdgpu_buffer_rsrc_t rs = r3d_rsrc(scale, s_bytes);
    const AnyBuf rsa = any_buf(scale, s_bytes);       /* the dword walk's view of the plane */
    auto sload = [&](uint32_t off) -> float {
        return UA ? lg_scale_any<SDT>(rsa, off) : lg_scale<SDT>(rs, off);
    };
    /* table value i of chunk k: row 16 chunk + i % 16, block i / 16 (zero past N and K) */
    auto tab_off = [&](int k, int i) -> uint32_t {
        const int64_t row = (ch0 + (int64_t)k * stride) * 16 + (i & 15);
        const int b = i >> 4;
        return k < nch && row < N && b < nwin ? (uint32_t)(((row / br) * s_pitch + b) * ESZ)
                                              : kLgOob;
    };
    auto tab_sync = [&](int k, float* tab, int from) {   /* values from..end, loaded and written */
        for (int i = from + l; i < 16 * nb_pad; i += 64) tab[i] = sload(tab_off(k, i));
    };
    /* how chunk k's scales are fetched: 1 by 16-byte unit, 2 one scale row by element, 0 by
     * table value (wave-uniform) */
    const int64_t span = 16 * s_pitch * ESZ;          /* a full chunk's rows, per-row grid */
    const int nunits = (int)(span / 16);
    auto tab_kind = [&](int k) -> int {
        if (k >= nch) return 0;
        if (br != 1) return 2;
        if (UA) return 0;
        const int64_t row0 = (ch0 + (int64_t)k * stride) * 16;
        if (N - row0 < 16 || (span & 15) || nunits > 64 * kLgTU ||
            ((reinterpret_cast<uintptr_t>(scale) + row0 * s_pitch * ESZ) & 15))
            return 0;
        return 1;
    };
    auto tab_fetch = [&](int k, r3d_i32x4* tu) __attribute__((always_inline)) {
        const int kind = tab_kind(k);
        const int64_t row0 = (ch0 + (int64_t)k * stride) * 16;
#pragma unroll
        for (int j = 0; j < kLgTU; ++j) tu[j] = r3d_i32x4{0, 0, 0, 0};
        if (kind == 1) {
#pragma unroll
            for (int j = 0; j < kLgTU; ++j) {
                const int u = l + 64 * j;
                tu[j] = r3d_buf_ld16_stream(rs, u < nunits ? (uint32_t)(row0 * s_pitch * ESZ + 16 * u)
                                                           : kLgOob);
            }
        } else if (kind == 2) {
            const int64_t srow = row0 / br;
#pragma unroll
            for (int j = 0; j < 4 * kLgTU; ++j) {
                const int b = l + 64 * j;
                if (64 * j < nwin)
                    tu[j >> 2][j & 3] = __float_as_int(
                        sload(b < nwin ? (uint32_t)((srow * s_pitch + b) * ESZ) : kLgOob));
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4 * kLgTU; ++j)
                if (64 * j < 16 * nb_pad)
                    tu[j >> 2][j & 3] = __float_as_int(sload(tab_off(k, l + 64 * j)));
        }
    };
    auto tab_write = [&](int k, const r3d_i32x4* tu) __attribute__((always_inline)) {
        const int kind = tab_kind(k);
        if (kind == 1) {
            constexpr int EPU = 16 / ESZ;             /* elements a unit */
            const int sp = (int)s_pitch;
#pragma unroll
            for (int j = 0; j < kLgTU; ++j) {
                const int u = l + 64 * j;
                if (u >= nunits) continue;
                int e = EPU * u, row = e / sp, b = e - row * sp;
#pragma unroll
                for (int i = 0; i < EPU; ++i) {
                    if (b < nwin) tab[16 * b + row] = lg_unit_elem<SDT>(tu[j], i);
                    if (++b == sp) { b = 0; ++row; }
                }
            }
        } else if (kind == 2) {
#pragma unroll
            for (int j = 0; j < 4 * kLgTU; ++j) {
                const int b = l + 64 * j;
                if (64 * j < nb_pad && b < nb_pad) {
                    const float v = __int_as_float(tu[j >> 2][j & 3]);
                    r3d_f32x4* t = reinterpret_cast<r3d_f32x4*>(tab + 16 * b);
                    t[0] = t[1] = t[2] = t[3] = r3d_f32x4{v, v, v, v};
                }
            }
            if (nb_pad > 64 * 4 * kLgTU) {            /* per-128-rows grids of very long K */
                const int64_t srow = ((ch0 + (int64_t)k * stride) * 16) / br;
                for (int b = 64 * 4 * kLgTU + l; b < nb_pad; b += 64) {
                    const float v = sload(b < nwin ? (uint32_t)((srow * s_pitch + b) * ESZ)
                                                   : kLgOob);
                    r3d_f32x4* t = reinterpret_cast<r3d_f32x4*>(tab + 16 * b);
                    t[0] = t[1] = t[2] = t[3] = r3d_f32x4{v, v, v, v};
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4 * kLgTU; ++j)
                if (64 * j + l < 16 * nb_pad) tab[64 * j + l] = __int_as_float(tu[j >> 2][j & 3]);
            if (16 * nb_pad > 64 * 4 * kLgTU) tab_sync(k, tab, 64 * 4 * kLgTU);
        }
    };

    /* the load cursor: chunk lk, window lw */
    const int kl = 64 * slot + 16 * kq;
    int lk = 0, lw = 0;
    r3d_i32x4 cb[RS][4];                              /* stream window t sits in slot t % RS */
    auto issue = [&](r3d_i32x4* dst) __attribute__((always_inline)) {
        const int64_t row0 = (ch0 + (int64_t)lk * stride) * 16;
        const int64_t rows_here = lk >= nch ? 0 : (N - row0 < 16 ? N - row0 : 16);
        const uint8_t* cbase = codes + (lk >= nch ? 0 : row0 * K);
        const int k = 256 * lw + kl;
        if (UA) {
            /* dword loads funnel-shifted; the bytes past K of a row (a partial piece: K is a
             * multiple of 4, k of 16) are zeroed, as are rows past the chunk's */
            const AnyBuf cu = any_buf(cbase, rows_here * K);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const bool in = k < K && 4 * g + lr < rows_here;
                r3d_i32x4 v = any_ld16(cu, in ? (uint32_t)((4 * g + lr) * K + k) : kAnyOob, false);
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (k + 4 * j >= K) v[j] = 0;
                dst[g] = v;
            }
        } else {
            const __amdgpu_buffer_rsrc_t rc = r3d_rsrc(cbase, rows_here * K);
#pragma unroll
            for (int g = 0; g < 4; ++g)
                dst[g] = r3d_buf_ld16_stream(rc, k < K ? (uint32_t)((4 * g + lr) * K + k) : kLgOob);
        }
        if (++lw == nw_pad) { lw = 0; ++lk; }
    };
#pragma unroll
    for (int d = 0; d < D; ++d) issue(cb[d]);
    tab_sync(0, tab, 0);
    if (tab_kind(0) == 1)                             /* keep the never-written blocks zero */
        for (int i = l; i < 16 * nb_pad; i += 64) tab[i] = (i >> 4) < nwin ? tab[i] : 0.0f;

    const uint8_t* xl = lg_lds + 2 * kl;              /* + x row * xrow + 512 w + 16 h */
    for (int k = 0; k < nch; ++k) {
        r3d_i32x4 tu[kLgTU];                          /* the next chunk's scales */
        tab_fetch(k + 1, tu);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   /* this chunk's table is written */
        r3d_f32x4 tot[XG][4];
#pragma unroll
        for (int xg = 0; xg < XG; ++xg)
#pragma unroll
            for (int g = 0; g < 4; ++g) tot[xg][g] = r3d_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        for (int w0 = 0; w0 < nw_pad; w0 += RS) {
#pragma unroll
            for (int j = 0; j < RS; ++j) {
                const int w = w0 + j;
                issue(cb[(j + D) % RS]);
                lg_bf16x8 xa[XG][2];
#pragma unroll
                for (int xg = 0; xg < XG; ++xg) {
                    xa[xg][0] = lg_bf16x8{};
                    xa[xg][1] = lg_bf16x8{};
                    if (4 * xg + lr < live) {
                        const uint8_t* xp = xl + (4 * xg + lr) * xrow + 512 * w;
                        xa[xg][0] = *reinterpret_cast<const lg_bf16x8*>(xp);
                        xa[xg][1] = *reinterpret_cast<const lg_bf16x8*>(xp + 16);
                    }
                }
                const float* st = tab + 16 * (2 * w + (kq >> 1));   /* used lanes: kq == slot */
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const r3d_i32x4 c = cb[j][g];
                    const lg_bf16x8 c0 = lg_codes8(c[0], c[1]), c1 = lg_codes8(c[2], c[3]);
                    const r3d_f32x4 sv = *reinterpret_cast<const r3d_f32x4*>(st + 4 * g);
#pragma unroll
                    for (int xg = 0; xg < XG; ++xg) {
                        const r3d_f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
                        r3d_f32x4 blk = __builtin_amdgcn_mfma_f32_16x16x32_bf16(c0, xa[xg][0], z, 0, 0, 0);
                        blk = __builtin_amdgcn_mfma_f32_16x16x32_bf16(c1, xa[xg][1], blk, 0, 0, 0);
#pragma unroll
                        for (int v = 0; v < 4; ++v) tot[xg][g][v] = fmaf(sv[v], blk[v], tot[xg][g][v]);
                    }
                }
            }
        }
        /* lanes t = 0..3 sum the slot lanes 20 s + t in slot order and store head rows
         * 16 chunk + 4 g + v */
        const int64_t row0 = (ch0 + (int64_t)k * stride) * 16;
#pragma unroll
        for (int xg = 0; xg < XG; ++xg)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                r3d_f32x4 o;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float t0 = tot[xg][g][v];
                    const float t1 = __shfl(t0, (l + 20) & 63, 64);
                    const float t2 = __shfl(t0, (l + 40) & 63, 64);
                    const float t3 = __shfl(t0, (l + 60) & 63, 64);
                    o[v] = ((t0 + t1) + t2) + t3;
                }
                const int m = 4 * xg + l;
                if (l < 4 && m < live) {
                    float* yp = Y + (int64_t)(mb + m) * y_pitch + row0 + 4 * g;
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        if (row0 + 4 * g + v < N) yp[v] = o[v];
                }
            }
        /* every read of this chunk's table has been consumed: the next chunk's goes in its
         * place */
        if (k + 1 < nch) tab_write(k + 1, tu);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   /* the loads past the last chunk */
}

/* ------------------------------------------------------------------ the blob's header */

/* Host copies of device-resident headers, per (device, blob): the first launch over a
 * blob in device memory reads its header and entries with a copy on the launch stream,
 * later launches reuse them (and the kernel re-checks them against the device copy before
 * reading a plane).  A blob in host-accessible memory is read in place every launch. */
struct HeadCacheEntry {
    int dev;
    const void* blob;
    RadPlanesHead h;
};
static std::mutex g_head_mu;
static HeadCacheEntry g_head[16];
static int g_head_n = 0, g_head_next = 0;

/* Where a blob lives: 1 host memory the device can read too (pinned, managed), 2 device
 * memory, 0 anything else -- ordinary host memory HIP does not know (also when no device
 * is present), readable by the host only -- and -1 for null. */
static int blob_kind(const void* blob) {
    if (!blob) return -1;
    hipPointerAttribute_t at;
    memset(&at, 0, sizeof at);
    if (hipPointerGetAttributes(&at, blob) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    if (at.type == hipMemoryTypeHost || at.type == hipMemoryTypeManaged ||
        at.type == hipMemoryTypeUnified)
        return 1;
    return at.type == hipMemoryTypeDevice || at.type == hipMemoryTypeArray ? 2 : 0;
}

/* The header, then its entries, read in place from host-readable memory; false for a
 * null blob.  Entries are read only for the two-plane header the plan accepts: a header
 * announcing any other count is refused without reading past the entries a two-plane blob
 * is sure to hold (the blob's extent is not known here). */
static bool head_read_host(const void* blob, RadPlanesHead* out) {
    if (!blob) return false;
    memset(out, 0, sizeof *out);
    memcpy(&out->h, blob, sizeof out->h);
    const RadPlanesHeader* h = rad_planes_header(blob);
    if (h && h->n_planes == 2) memcpy(out->e, rad_planes_entries(h), 2 * sizeof(RadPlanesEntry));
    return true;
}

static bool head_cached(int dev, const void* blob, RadPlanesHead* out) {
    std::lock_guard<std::mutex> lk(g_head_mu);
    for (int i = 0; i < g_head_n; ++i)
        if (g_head[i].dev == dev && g_head[i].blob == blob) {
            *out = g_head[i].h;
            return true;
        }
    return false;
}

/* The launch's view of the header: in place, cached, or (first launch over a device blob)
 * copied on `stream` -- the header, then the entries it announces -- and synchronised, so
 * the copy is ordered after the stream's earlier writes to the blob.  A first launch under
 * graph capture is refused (RAD_E_UNSUPPORTED): the copy and the wait cannot be captured. */
static int head_copy(const void* blob, hipStream_t stream, RadPlanesHead* out) {
    const int kind = blob_kind(blob);
    if (kind == 1) return head_read_host(blob, out) && rad_planes_header(blob) ? RAD_OK : RAD_E_DTYPE;
    if (kind != 2) return RAD_E_DTYPE;          /* the kernel could not read it */
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return RAD_E_DEVICE;
    if (head_cached(dev, blob, out)) return RAD_OK;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) != hipSuccess) {
        (void)hipGetLastError();
        return RAD_E_DEVICE;
    }
    if (cs != hipStreamCaptureStatusNone) {
        fprintf(stderr, "libr3d_gfx950: logits_gemm_e4m3: the first launch over a device-"
                        "resident head is under graph capture; launch once before capturing\n");
        return RAD_E_UNSUPPORTED;
    }
    memset(out, 0, sizeof *out);
    if (hipMemcpyAsync(&out->h, blob, sizeof out->h, hipMemcpyDeviceToHost, stream) != hipSuccess ||
        hipStreamSynchronize(stream) != hipSuccess) {
        (void)hipGetLastError();
        return RAD_E_DEVICE;
    }
    /* two planes or none: the copy never reaches past what a two-plane blob holds */
    if (!rad_planes_header(&out->h) || out->h.n_planes != 2) return RAD_E_DTYPE;
    if (hipMemcpyAsync(out->e, rad_planes_entries(reinterpret_cast<const RadPlanesHeader*>(blob)),
                       2 * sizeof(RadPlanesEntry), hipMemcpyDeviceToHost,
                       stream) != hipSuccess ||
        hipStreamSynchronize(stream) != hipSuccess) {
        (void)hipGetLastError();
        return RAD_E_DEVICE;
    }
    std::lock_guard<std::mutex> lk(g_head_mu);
    HeadCacheEntry& e = g_head[g_head_n < 16 ? g_head_n++ : (g_head_next++ & 15)];
    e.dev = dev;
    e.blob = blob;
    e.h = *out;
    return RAD_OK;
}

static void head_forget(const void* blob) {
    std::lock_guard<std::mutex> lk(g_head_mu);
    int j = 0;
    for (int i = 0; i < g_head_n; ++i)
        if (g_head[i].blob != blob) g_head[j++] = g_head[i];
    g_head_n = j;
    g_head_next = 0;
}

bool logits_head_peek(const void* blob, RadPlanesHead* out) {
    const int kind = blob_kind(blob);
    if (kind == 0 || kind == 1) return head_read_host(blob, out);
    int dev = 0;
    return kind == 2 && hipGetDevice(&dev) == hipSuccess && head_cached(dev, blob, out);
}

/* ---------------------------------------------------------------------- the row entry */

/* Workgroups of `waves` waves of this instantiation one compute unit holds at `lds` bytes
 * of LDS (the register count answered once by the runtime). */
template <int D, int XG, int SDT, bool UA>
static int logits_per_cu(int waves, int lds) {
    static int regs[9];
    if (!regs[waves]) {
        (void)hipFuncSetAttribute(
            reinterpret_cast<const void*>(&logits_e4m3_kernel<D, XG, SDT, UA>),
            hipFuncAttributeMaxDynamicSharedMemorySize, kLogitsLds);
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &n, reinterpret_cast<const void*>(&logits_e4m3_kernel<D, XG, SDT, UA>),
                waves * 64, 0) != hipSuccess || n < 1)
            n = 1;
        (void)hipGetLastError();
        regs[waves] = n;
    }
    const int by_lds = lds > 0 ? kLogitsLds / lds : regs[waves];
    const int n = by_lds < regs[waves] ? by_lds : regs[waves];
    return n < 1 ? 1 : n;
}

template <int D, int XG, int SDT, bool UA>
static hipError_t launch_logits_t(const LogitsPlan& P, hipStream_t stream) {
    const LogitsGeom g = logits_geom(P, cu_count(), logits_per_cu<D, XG, SDT, UA>(P.waves, P.lds));
    const int esz = SDT == 2 ? 4 : 2;
    const int64_t s_bytes = P.guard.s_rows * P.s_pitch * esz;
    hipLaunchKernelGGL((logits_e4m3_kernel<D, XG, SDT, UA>),
                       dim3((unsigned)g.blocks, (unsigned)g.passes), dim3(P.waves * 64),
                       (size_t)P.lds, stream, P.X, P.x_pitch, P.codes, P.scale, P.s_pitch,
                       s_bytes, P.br, P.Y, P.y_pitch, (int)P.N, (int)P.K, (int)P.M, P.mt,
                       P.nwin, P.nw_pad, P.xrow, P.mt * P.xrow, g.chunks, P.guard);
    return hipGetLastError();
}

template <int D, int XG, bool UA>
static hipError_t launch_logits_dx(const LogitsPlan& P, hipStream_t s) {
    return P.sdt == 0 ? launch_logits_t<D, XG, 0, UA>(P, s)
         : P.sdt == 1 ? launch_logits_t<D, XG, 1, UA>(P, s)
                      : launch_logits_t<D, XG, 2, UA>(P, s);
}

template <bool UA>
static hipError_t launch_logits_u(const LogitsPlan& P, hipStream_t stream) {
    /* 5..8 activation rows a pass: two groups of 4, one window in flight (the plan's rule) */
    return P.mt > 4        ? launch_logits_dx<1, 2, UA>(P, stream)
         : P.depth == 3    ? launch_logits_dx<3, 1, UA>(P, stream)
         : P.depth == 2    ? launch_logits_dx<2, 1, UA>(P, stream)
                           : launch_logits_dx<1, 1, UA>(P, stream);
}

static int logits_entry(const RadArgs* a, RadStream s) {
    LogitsPlan P{};
    int rc = plan_logits_e4m3(a, nullptr, &P, true);
    if (rc) return rc;
    if (!chip_ok()) return RAD_E_UNSUPPORTED;
    hipStream_t stream = (hipStream_t)s;
    RadPlanesHead hc;
    rc = head_copy(rad_arg_in(a, 1)->data, stream, &hc);
    if (rc) return rc;
    rc = plan_logits_e4m3(a, &hc, &P, false);
    if (rc) return rc;
    const hipError_t e = P.ua ? launch_logits_u<true>(P, stream) : launch_logits_u<false>(P, stream);
    if (e != hipSuccess) {
        fprintf(stderr, "libr3d_gfx950: logits_e4m3 launch FAILED (%s)\n", hipGetErrorName(e));
        return RAD_E_DEVICE;
    }
    return RAD_OK;
}

}  // namespace r3d

extern "C" {

int r3d_rad_logits_gemm_e4m3(const RadArgs* a, RadStream s) {
    return r3d::dump_wrap("logits_gemm_e4m3", a, s, r3d::logits_entry);
}

void r3d_gfx950_logits_head_forget(const void* blob) { r3d::head_forget(blob); }

}  /* extern "C" */
