/* r3d_noalloc.hip -- gemm_nt_q_mxfp4a16 without caller scratch, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).
 *
 * The mxfp4a16 row quantises its bf16 activations into launch scratch (e4m3 codes, then
 * E8M0 scales) before the GEMM reads them.  This entry runs the same kernels with that
 * scratch in a file-scope device array of R3D_NOALLOC_SCRATCH_BYTES: each GPU the library
 * runs on holds its own copy until the process ends, and the entry allocates and frees
 * nothing.  Every call on one GPU shares that GPU's array, so calls that overlap on one
 * GPU (two streams, two threads) race on it; calls in one stream order are safe.  The
 * quantiser writes every byte the GEMM then reads, so nothing has to start at zero.
 */
#include <hip/hip_runtime.h>

#include <mutex>
#include <stdio.h>
#include <string.h>

#include "r3d_gfx950.h"
#include "r3d_plan.h"
#include "rad_plugin.h"

/* The static scratch.  In host code this name is only a handle for the symbol lookup
 * below: its device address is taken once per device with hipGetSymbolAddress and only
 * that address is ever handed to a kernel. */
static __device__ __align__(256) uint8_t scratch[R3D_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;

/* The current device's copy of `scratch`, set up on the first call on that device (with
 * it current) and kept: RAD_OK and *out, RAD_E_UNSUPPORTED on a device that is not gfx950
 * (the library holds gfx950 code objects only), RAD_E_DEVICE if the lookup fails. */
int device_scratch(uint8_t** out) {
    static std::mutex mu;
    static uint8_t* ptr[kMaxDevices];
    static int state[kMaxDevices];               /* 0 not set up, 1 ready, 2 not gfx950 */
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return RAD_E_DEVICE;
    std::lock_guard<std::mutex> lock(mu);
    if (state[dev] == 0) {
        hipDeviceProp_t prop;
        memset(&prop, 0, sizeof prop);
        if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return RAD_E_DEVICE;
        if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
            state[dev] = 2;
        } else {
            void* p = nullptr;
            const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess || !p) {
                fprintf(stderr, "libr3d_gfx950: mxfp4a16_noalloc: scratch lookup on device %d "
                                "FAILED (%s)\n", dev, hipGetErrorName(e));
                return RAD_E_DEVICE;
            }
            ptr[dev] = static_cast<uint8_t*>(p);
            state[dev] = 1;
        }
    }
    if (state[dev] != 1) return RAD_E_UNSUPPORTED;
    *out = ptr[dev];
    return RAD_OK;
}

}  // namespace

extern "C" int r3d_rad_gemm_nt_q_mxfp4a16_noalloc(const RadArgs* a, RadStream s) {
    if (!a) return RAD_E_INVAL;
    if (r3d::env_no_mxfp4()) return RAD_E_UNSUPPORTED;
    /* the scratch this call needs: M = numel(y) / N rows of K */
    int64_t M = 0, N = 0;
    const int rc = r3d::entry_preamble(a, r3d::ENC_MXFP4A16, 0, &M, &N);
    if (rc) return rc;
    long long K = 0;
    if (!rad_args_geti(a, "K", &K) || K <= 0) return RAD_E_SHAPE;
    const int64_t need = r3d::mxfp4a16_scratch_bytes(M, K);
    if (need < 0) return RAD_E_SHAPE;                 /* M or K past any plan's bound */
    if (need > (int64_t)R3D_NOALLOC_SCRATCH_BYTES) {
        fprintf(stderr, "libr3d_gfx950: mxfp4a16_noalloc: M=%lld K=%lld needs %lld bytes of "
                        "scratch, the static buffer holds %lld (refused)\n",
                (long long)M, K, (long long)need, (long long)R3D_NOALLOC_SCRATCH_BYTES);
        return RAD_E_SHAPE;
    }
    uint8_t* p = nullptr;
    const int st = device_scratch(&p);
    if (st) return st;
    RadArgs b = *a;
    b.scratch = p;
    b.scratch_bytes = R3D_NOALLOC_SCRATCH_BYTES;
    return r3d_rad_gemm_nt_q_mxfp4a16(&b, s);
}
