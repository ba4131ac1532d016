/* r3d_probe.hip -- measurement diagnostics with no counterpart in the reference: the
 * ceilings the decode GEMVs are held against (bench.py --floors).
 *
 *   r3d_gfx950_stream_probe: a read-only stream over `bytes` of device memory, each wave
 *   reading its own contiguous run of `kb` KB with 1 KB loads (64 lanes x 16 bytes,
 *   non-temporal, the GEMVs' load instruction) kept 8 deep in flight, the bytes XOR-folded
 *   into a register that is stored only if it equals a value the data never produces (so no
 *   load can be dropped); bytes = 0 launches `waves` waves that do nothing (the launch
 *   floor).  Nothing else rides the vector-memory queue, so its time is what the access
 *   pattern alone costs at that size.
 */
#include <hip/hip_runtime.h>

#include <stdio.h>

#include "r3d_device.h"
#include "rad_abi.h"

namespace r3d {

constexpr int kProbeDepth = 8;

__global__ __launch_bounds__(512) void stream_probe_kernel(const uint8_t* src, int64_t bytes,
                                                           int run, uint32_t* sink) {
    const int lane = threadIdx.x & 63;
    const int64_t w = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int64_t base = w * (int64_t)run;
    if (bytes == 0 || base >= bytes) return;
    const int64_t left = bytes - base;
    const int n = (int)((left < run ? left : run) >> 10);          /* whole 1 KB loads */
    const __amdgpu_buffer_rsrc_t r = r3d_rsrc(src + base, left < run ? left : run);
    uint32_t acc = 0;
    r3d_i32x4 ring[kProbeDepth];
#pragma unroll
    for (int d = 0; d < kProbeDepth; ++d)
        ring[d] = r3d_buf_ld16_stream(r, d < n ? (uint32_t)(1024 * d + 16 * lane) : 0x80000000u);
    for (int i = 0; i < n; i += kProbeDepth) {
#pragma unroll
        for (int d = 0; d < kProbeDepth; ++d) {
            acc ^= (uint32_t)(ring[d][0] ^ ring[d][1] ^ ring[d][2] ^ ring[d][3]);
            const int nx = i + kProbeDepth + d;
            ring[d] = r3d_buf_ld16_stream(r, nx < n ? (uint32_t)(1024 * nx + 16 * lane)
                                                    : 0x80000000u + 16 * d);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

}  // namespace r3d

extern "C" int r3d_gfx950_stream_probe(const void* src, int64_t bytes, int waves_per_wg,
                                       int64_t kb, uint32_t* sink, RadStream s) {
    if (bytes < 0 || kb < 1 || kb > (1 << 20) || waves_per_wg < 1 || waves_per_wg > 8 || !sink)
        return RAD_E_INVAL;
    const int64_t run = kb * 1024;
    const int64_t waves = bytes > 0 ? (bytes + run - 1) / run : kb;   /* bytes 0: kb waves */
    const int64_t blocks = (waves + waves_per_wg - 1) / waves_per_wg;
    if (blocks > 0x7FFFFFFF || run > 0x7FFFFFFF) return RAD_E_SHAPE;
    hipLaunchKernelGGL(r3d::stream_probe_kernel, dim3((unsigned)blocks), dim3(64 * waves_per_wg),
                       0, (hipStream_t)s, (const uint8_t*)src, bytes, (int)run, sink);
    return hipGetLastError() == hipSuccess ? RAD_OK : RAD_E_DEVICE;
}
