/* r3d_logits.hip -- the gfx950 logits_gemm_e4m3 row: logits over a joined e4m3 +
 * block-scale lm_head (the reference's row is src/r3d_gemm_logits.hip:72-226, its layout
 * hooks :233-272).
 *
 *     y[m, n] = sum_k x[m, k] * e4m3(codes[n, k]) * scale[n / br, k / 128]     (f32 out)
 *
 * On MFMA.  A decoded e4m3 code has 4 significant bits and an exponent inside bf16's range,
 * so it is exact in bf16 (v_cvt_scalef32_pk_bf16_fp8 at scale 1 reproduces all 256 codes,
 * NaN included); x is bf16 already.  v_mfma_f32_16x16x32_bf16 therefore forms every product
 * x * code exactly -- 8 x 4 significant bits -- and sums 32 of them at f32 accuracy (worst
 * measured on MI355X: 5.9 * 2^-24 of the sum of magnitudes per instruction, C included).
 * The scale, which need not be a power of two, is applied once per 128-wide window, in f32:
 * tot = fma(scale, window_sum, tot).  This differs from the reference's order (one fma per
 * product, code * scale rounded first) only in where the f32 roundings fall; both stay
 * within (window count + 4 * 66) * 2^-24 * sum |x * code * scale| of the exact sum.
 *
 * Layout of one step (a 128-wide K window, w):
 *   A = 16 activation rows, staged once per workgroup in LDS as bf16 (rows mb .. mb+mt,
 *       zero past K up to a multiple of 4 windows), lane (m = l%16, q = l/16) reading its
 *       row's columns [128w + 16q, +16) and [128w + 64 + 16q, +16);
 *   B = 16 head rows streamed from HBM: lane (r = l%16, q) loads 16 code bytes of row r at
 *       each of those two column ranges (buffer loads: a chunk past K or a row past N reads
 *       zero), and each 8-byte half feeds one of the four MFMAs of the window;
 *   D = lane (r, q) holds x rows 4q .. 4q+3 for head row r, so its four accumulators share
 *       one scale: lane (r, q) loads row r's scale for window 4t + q once every four windows
 *       and the window's value comes from lane r + 16 (w % 4) by one ds_bpermute.
 * A wave owns G groups of 16 head rows (a chunk), so one A fragment from LDS feeds G x 4
 * MFMAs; chunks are dealt to waves blocks * 8 apart.  The codes of window w + 1 are in
 * flight while window w computes.  Bytes per head row: K codes + 2 or 4 per 128 columns
 * of scale (br = 1) -- the kernel is bound by HBM, the MFMAs run at a few percent.
 */
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <mutex>
#include <stdio.h>
#include <string.h>

#include "r3d_device.h"
#include "r3d_dump.h"
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

/* The device copy of the header still describes the planes the host planned from. */
__device__ __forceinline__ bool lg_header_ok(const LogitsGuard& g) {
    const RadPlanesHeader* h = reinterpret_cast<const RadPlanesHeader*>(g.header);
    if (h->magic != RAD_PLANES_MAGIC || h->version != RAD_PLANES_VERSION || h->n_planes != 2)
        return false;
    const RadPlanesEntry& c = h->entry[g.ic];
    const RadPlanesEntry& s = h->entry[g.is];
    return c.dtype == RAD_F8E4M3 && c.offset == g.c_off && c.rows == g.c_rows &&
           c.cols == g.c_cols && s.dtype == g.s_dtype && s.offset == g.s_off &&
           s.rows == g.s_rows && s.row_bytes == g.s_row_bytes && s.block[0] == g.s_br;
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

template <int D, int XG, int SDT>
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
        if (8 * c < K) v = *reinterpret_cast<const r3d_i32x4*>(X + (int64_t)(mb + m) * x_pitch + 8 * c);
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
    /* table value i of chunk k: row 16 chunk + i % 16, block i / 16 (zero past N and K) */
    auto tab_off = [&](int k, int i) -> uint32_t {
        const int64_t row = (ch0 + (int64_t)k * stride) * 16 + (i & 15);
        const int b = i >> 4;
        return k < nch && row < N && b < nwin ? (uint32_t)(((row / br) * s_pitch + b) * ESZ)
                                              : kLgOob;
    };
    auto tab_sync = [&](int k, float* tab, int from) {   /* values from..end, loaded and written */
        for (int i = from + l; i < 16 * nb_pad; i += 64) tab[i] = lg_scale<SDT>(rs, tab_off(k, i));
    };
    /* how chunk k's scales are fetched: 1 by 16-byte unit, 2 one scale row by element, 0 by
     * table value (wave-uniform) */
    const int64_t span = 16 * s_pitch * ESZ;          /* a full chunk's rows, per-row grid */
    const int nunits = (int)(span / 16);
    auto tab_kind = [&](int k) -> int {
        if (k >= nch) return 0;
        if (br != 1) return 2;
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
                    tu[j >> 2][j & 3] = __float_as_int(lg_scale<SDT>(
                        rs, b < nwin ? (uint32_t)((srow * s_pitch + b) * ESZ) : kLgOob));
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4 * kLgTU; ++j)
                if (64 * j < 16 * nb_pad)
                    tu[j >> 2][j & 3] = __float_as_int(lg_scale<SDT>(rs, tab_off(k, l + 64 * j)));
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
                    const float v = lg_scale<SDT>(rs, b < nwin ? (uint32_t)((srow * s_pitch + b) * ESZ)
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
        const __amdgpu_buffer_rsrc_t rc = r3d_rsrc(codes + (lk >= nch ? 0 : row0 * K), rows_here * K);
        const int k = 256 * lw + kl;
#pragma unroll
        for (int g = 0; g < 4; ++g)
            dst[g] = r3d_buf_ld16_stream(rc, k < K ? (uint32_t)((4 * g + lr) * K + k) : kLgOob);
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
 * blob in device memory reads its header with one synchronous copy, later launches reuse
 * it (and the kernel re-checks it against the device copy before reading a plane).  A blob
 * in pinned or managed memory is read in place every launch. */
struct HeadCacheEntry {
    int dev;
    const void* blob;
    RadPlanesHeader h;
};
static std::mutex g_head_mu;
static HeadCacheEntry g_head[16];
static int g_head_n = 0, g_head_next = 0;

static bool head_copy(const void* blob, RadPlanesHeader* out) {
    if (!blob) return false;
    hipPointerAttribute_t at;
    memset(&at, 0, sizeof at);
    if (hipPointerGetAttributes(&at, blob) != hipSuccess) {
        (void)hipGetLastError();                      /* unregistered host memory */
        return false;
    }
    if (at.type == hipMemoryTypeHost || at.type == hipMemoryTypeManaged ||
        at.type == hipMemoryTypeUnified) {
        memcpy(out, blob, sizeof *out);
        return rad_planes_header(out) != nullptr;
    }
    if (at.type != hipMemoryTypeDevice) return false;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    {
        std::lock_guard<std::mutex> lk(g_head_mu);
        for (int i = 0; i < g_head_n; ++i)
            if (g_head[i].dev == dev && g_head[i].blob == blob) {
                *out = g_head[i].h;
                return true;
            }
    }
    if (hipMemcpy(out, blob, sizeof *out, hipMemcpyDeviceToHost) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    if (!rad_planes_header(out)) return false;
    std::lock_guard<std::mutex> lk(g_head_mu);
    HeadCacheEntry& e = g_head[g_head_n < 16 ? g_head_n++ : (g_head_next++ & 15)];
    e.dev = dev;
    e.blob = blob;
    e.h = *out;
    return true;
}

static void head_forget(const void* blob) {
    std::lock_guard<std::mutex> lk(g_head_mu);
    int j = 0;
    for (int i = 0; i < g_head_n; ++i)
        if (g_head[i].blob != blob) g_head[j++] = g_head[i];
    g_head_n = j;
    g_head_next = 0;
}

/* ---------------------------------------------------------------------- the row entry */

/* Workgroups of `waves` waves of this instantiation one compute unit holds at `lds` bytes
 * of LDS (the register count answered once by the runtime). */
template <int D, int XG, int SDT>
static int logits_per_cu(int waves, int lds) {
    static int regs[9];
    if (!regs[waves]) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&logits_e4m3_kernel<D, XG, SDT>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, kLogitsLds);
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &n, reinterpret_cast<const void*>(&logits_e4m3_kernel<D, XG, SDT>), waves * 64,
                0) != hipSuccess || n < 1)
            n = 1;
        (void)hipGetLastError();
        regs[waves] = n;
    }
    const int by_lds = lds > 0 ? kLogitsLds / lds : regs[waves];
    const int n = by_lds < regs[waves] ? by_lds : regs[waves];
    return n < 1 ? 1 : n;
}

template <int D, int XG, int SDT>
static hipError_t launch_logits_t(const LogitsPlan& P, hipStream_t stream) {
    const LogitsGeom g = logits_geom(P, cu_count(), logits_per_cu<D, XG, SDT>(P.waves, P.lds));
    const int esz = SDT == 2 ? 4 : 2;
    const int64_t s_bytes = P.guard.s_rows * P.s_pitch * esz;
    hipLaunchKernelGGL((logits_e4m3_kernel<D, XG, SDT>),
                       dim3((unsigned)g.blocks, (unsigned)g.passes), dim3(P.waves * 64),
                       (size_t)P.lds, stream, P.X, P.x_pitch, P.codes, P.scale, P.s_pitch,
                       s_bytes, P.br, P.Y, P.y_pitch, (int)P.N, (int)P.K, (int)P.M, P.mt,
                       P.nwin, P.nw_pad, P.xrow, P.mt * P.xrow, g.chunks, P.guard);
    return hipGetLastError();
}

template <int D, int XG>
static hipError_t launch_logits_dx(const LogitsPlan& P, hipStream_t s) {
    return P.sdt == 0 ? launch_logits_t<D, XG, 0>(P, s)
         : P.sdt == 1 ? launch_logits_t<D, XG, 1>(P, s)
                      : launch_logits_t<D, XG, 2>(P, s);
}


static int logits_entry(const RadArgs* a, RadStream s) {
    LogitsPlan P{};
    int rc = plan_logits_e4m3(a, nullptr, &P, true);
    if (rc) return rc;
    if (!chip_ok()) return RAD_E_UNSUPPORTED;
    RadPlanesHeader hc;
    if (!head_copy(rad_arg_in(a, 1)->data, &hc)) return RAD_E_DTYPE;
    rc = plan_logits_e4m3(a, &hc, &P, false);
    if (rc) return rc;
    hipStream_t stream = (hipStream_t)s;
    /* 5..8 activation rows a pass: two groups of 4, one window in flight (the plan's rule) */
    const hipError_t e = P.mt > 4        ? launch_logits_dx<1, 2>(P, stream)
                       : P.depth == 3    ? launch_logits_dx<3, 1>(P, stream)
                       : P.depth == 2    ? launch_logits_dx<2, 1>(P, stream)
                                         : launch_logits_dx<1, 1>(P, stream);
    if (e != hipSuccess) {
        fprintf(stderr, "libr3d_gfx950: logits_e4m3 launch FAILED (%s)\n", hipGetErrorName(e));
        return RAD_E_DEVICE;
    }
    return RAD_OK;
}

/* ------------------------------------------------------------------ joining the planes */

/* The joined head's layout (header, then the codes and the scale plane each at a 256-byte
 * boundary), written into *h when given; the blob's bytes, or minus a RAD_E_* code. */
static int64_t head_layout(int64_t N, int64_t K, uint32_t sdt, int64_t br, RadPlanesHeader* h) {
    if (N <= 0 || K <= 0 || N > 0x7FFFFFFLL || K > 0x7FFFFFFLL) return -RAD_E_SHAPE;
    if (sdt != RAD_BF16 && sdt != RAD_F16 && sdt != RAD_F32) return -RAD_E_DTYPE;
    if (br != 1 && br != 128) return -RAD_E_SHAPE;
    const int64_t esz = sdt == RAD_F32 ? 4 : 2;
    const int64_t srows = (N + br - 1) / br, scols = (K + 127) / 128;
    auto up = [](int64_t v) { return (v + 255) / 256 * 256; };
    const int64_t c_off = up((int64_t)sizeof(RadPlanesHeader));
    const int64_t s_off = up(c_off + N * K);
    if (h) {
        memset(h, 0, sizeof *h);
        h->magic = RAD_PLANES_MAGIC;
        h->version = RAD_PLANES_VERSION;
        h->n_planes = 2;
        RadPlanesEntry& c = h->entry[0];
        strncpy(c.role, "codes", RAD_PLANES_ROLE);
        c.dtype = RAD_F8E4M3;
        c.block[0] = 1; c.block[1] = 1;
        c.rows = N; c.cols = K; c.row_bytes = K; c.offset = c_off;
        RadPlanesEntry& e = h->entry[1];
        strncpy(e.role, "scale", RAD_PLANES_ROLE);
        e.dtype = sdt;
        e.block[0] = br; e.block[1] = 128;
        e.rows = srows; e.cols = scols; e.row_bytes = scols * esz; e.offset = s_off;
        h->bytes = s_off + srows * scols * esz;
    }
    return s_off + srows * scols * esz;
}

}  // namespace r3d

extern "C" {

int r3d_rad_logits_gemm_e4m3(const RadArgs* a, RadStream s) {
    return r3d::dump_wrap("logits_gemm_e4m3", a, s, r3d::logits_entry);
}

int64_t r3d_gfx950_logits_head_bytes(int64_t n_vocab, int64_t n_embd, uint32_t scale_dtype,
                                     int64_t scale_block_rows) {
    return r3d::head_layout(n_vocab, n_embd, scale_dtype, scale_block_rows, nullptr);
}

int64_t r3d_gfx950_logits_head_header(int64_t n_vocab, int64_t n_embd, uint32_t scale_dtype,
                                      int64_t scale_block_rows, RadPlanesHeader* out) {
    if (!out) return -RAD_E_INVAL;
    return r3d::head_layout(n_vocab, n_embd, scale_dtype, scale_block_rows, out);
}

int r3d_gfx950_logits_head_join(const uint8_t* codes, int64_t codes_pitch, const void* scale,
                                int64_t scale_pitch_bytes, int64_t n_vocab, int64_t n_embd,
                                uint32_t scale_dtype, int64_t scale_block_rows, void* dst,
                                int64_t dst_bytes) {
    RadPlanesHeader h;
    const int64_t need = r3d::head_layout(n_vocab, n_embd, scale_dtype, scale_block_rows, &h);
    if (need < 0) return (int)-need;
    if (!codes || !scale || !dst || dst_bytes < need) return RAD_E_SHAPE;
    const RadPlanesEntry& c = h.entry[0];
    const RadPlanesEntry& e = h.entry[1];
    if (codes_pitch < n_embd || scale_pitch_bytes < e.row_bytes) return RAD_E_STRIDE;
    uint8_t* d = (uint8_t*)dst;
    memset(d, 0, (size_t)need);
    memcpy(d, &h, sizeof h);
    for (int64_t i = 0; i < n_vocab; ++i)
        memcpy(d + c.offset + i * n_embd, codes + i * codes_pitch, (size_t)n_embd);
    for (int64_t i = 0; i < e.rows; ++i)
        memcpy(d + e.offset + i * e.row_bytes, (const uint8_t*)scale + i * scale_pitch_bytes,
               (size_t)e.row_bytes);
    return RAD_OK;
}

int r3d_gfx950_logits_head_split(const void* blob, int64_t blob_bytes, uint8_t* codes,
                                 void* scale) {
    if (!blob || blob_bytes < (int64_t)sizeof(RadPlanesHeader)) return RAD_E_SHAPE;
    const RadPlanesHeader* h = rad_planes_header(blob);
    const RadPlanesEntry* c = nullptr;
    const RadPlanesEntry* e = nullptr;
    if (!h || h->n_planes != 2 || !rad_planes_find(blob, "codes", &c) ||
        !rad_planes_find(blob, "scale", &e))
        return RAD_E_DTYPE;
    if (h->bytes > blob_bytes || c->offset + c->rows * c->row_bytes > h->bytes ||
        e->offset + e->rows * e->row_bytes > h->bytes)
        return RAD_E_SHAPE;
    const int64_t esz = e->dtype == RAD_F32 ? 4 : 2;
    const uint8_t* b = (const uint8_t*)blob;
    if (codes)
        for (int64_t i = 0; i < c->rows; ++i)
            memcpy(codes + i * c->cols, b + c->offset + i * c->row_bytes, (size_t)c->cols);
    if (scale)
        for (int64_t i = 0; i < e->rows; ++i)
            memcpy((uint8_t*)scale + i * e->cols * esz, b + e->offset + i * e->row_bytes,
                   (size_t)(e->cols * esz));
    return RAD_OK;
}

void r3d_gfx950_logits_head_forget(const void* blob) { r3d::head_forget(blob); }

}  /* extern "C" */
