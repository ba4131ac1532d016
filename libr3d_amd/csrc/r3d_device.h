/* r3d_device.h -- gfx950 device helpers shared by the gemm_nt_q kernels.
 *
 * Operand layouts of v_mfma_scale_f32_16x16x128_f8f6f4, as measured on MI355X (wave64,
 * lane l, hardware K index inside one 128-wide step):
 *   fp4 operand : lane (row l%16, q = l/16) holds K [32q, 32q+32), nibble p = K 32q+p,
 *                 low nibble first -- one whole 32-wide scale block per lane;
 *   fp8 operand : lane (row l%16, kb = l/16) holds K [16kb, 16kb+16) in bytes 0..15 and
 *                 K [64+16kb, 64+16kb+16) in bytes 16..31;
 *   scales      : the E8M0 byte for (row r, block b = K/32) is read from lane 16b + r of
 *                 the scale operand, independent of where that block's data sits;
 *   result      : lane l holds D[4*(l/16) + i][l%16] in element i (row of src A, column
 *                 of src B).
 * E8M0 0xFF yields NaN even when every product is zero, 0x00 is 2^-127 with f32
 * subnormals kept, and e4m3 subnormals / the S1111111 NaN are honoured -- the same
 * semantics as libref's e8m0_to_f32 / rad_fp8e4m3_to_f32.
 */
#ifndef R3D_DEVICE_H
#define R3D_DEVICE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef int   r3d_i32x8 __attribute__((ext_vector_type(8)));
typedef int   r3d_i32x4 __attribute__((ext_vector_type(4)));
typedef float r3d_f32x4 __attribute__((ext_vector_type(4)));

enum { R3D_MFMA_FP8 = 0, R3D_MFMA_FP4 = 4 };
enum { R3D_E8M0_ONE = 127 };

/* D = A(16 x 128, fp4, scale per lane) . B(16 x 128, fp8)^T, fresh accumulator. */
__device__ __forceinline__ r3d_f32x4 r3d_mfma_fp4_fp8(r3d_i32x4 a, int scale_a, r3d_i32x8 b,
                                                      int scale_b) {
    const r3d_i32x8 a8 = {a[0], a[1], a[2], a[3], 0, 0, 0, 0};
    const r3d_f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a8, b, z, R3D_MFMA_FP4, R3D_MFMA_FP8,
                                                            0, scale_a, 0, scale_b);
}

/* C += A(16 x 128, fp4, scale per lane) . B(16 x 128, fp8, scale per lane)^T. */
__device__ __forceinline__ r3d_f32x4 r3d_mfma_fp4_fp8_acc(r3d_i32x4 a, int scale_a, r3d_i32x8 b,
                                                          int scale_b, r3d_f32x4 c) {
    const r3d_i32x8 a8 = {a[0], a[1], a[2], a[3], 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a8, b, c, R3D_MFMA_FP4, R3D_MFMA_FP8,
                                                            0, scale_a, 0, scale_b);
}

/* Direct global -> LDS load of `bytes` (16, 4 or 2) per lane: lane l's data lands at
 * lds + l * max(bytes, 4); the LDS base must be wave-uniform. */
__device__ __forceinline__ void r3d_lds_load(const void* g, void* l, int bytes) {
    if (bytes == 16)
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)g,
                                         (__attribute__((address_space(3))) void*)l, 16, 0, 0);
    else if (bytes == 4)
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)g,
                                         (__attribute__((address_space(3))) void*)l, 4, 0, 0);
    else
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)g,
                                         (__attribute__((address_space(3))) void*)l, 2, 0, 0);
}

/* D = A(16 x 128, fp8) . B(16 x 128, fp8)^T, unit scales, fresh accumulator. */
__device__ __forceinline__ r3d_f32x4 r3d_mfma_fp8_fp8(r3d_i32x8 a, r3d_i32x8 b) {
    const r3d_f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, R3D_MFMA_FP8, R3D_MFMA_FP8,
                                                            0, R3D_E8M0_ONE, 0, R3D_E8M0_ONE);
}

/* 16-byte global load (global_load_dwordx4); the address must be 16-byte aligned. */
__device__ __forceinline__ r3d_i32x4 r3d_ld16(const uint8_t* p) {
    return *reinterpret_cast<const r3d_i32x4*>(p);
}

/* Non-temporal 16-byte load for bytes read exactly once per call (weight planes). */
__device__ __forceinline__ r3d_i32x4 r3d_ld16_stream(const uint8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const r3d_i32x4*>(p));
}

/* Buffer resource over [base, base + bytes) (raw, stride 0): loads past `bytes` read 0. */
__device__ __forceinline__ __amdgpu_buffer_rsrc_t r3d_rsrc(const void* base, int64_t bytes) {
    const int n = bytes > 0x7FFFFFFF ? 0x7FFFFFFF : (int)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}

/* Buffer load of `bytes` (16, 4 or 2) per lane straight into LDS at lds + lane *
 * max(bytes, 4). */
template <int BYTES>
__device__ __forceinline__ void r3d_buf_lds(__amdgpu_buffer_rsrc_t r, uint8_t* lds, uint32_t voff,
                                            uint32_t soff) {
    static_assert(BYTES == 16 || BYTES == 4 || BYTES == 2, "dwordx4, dword or ushort loads");
    if constexpr (BYTES == 16)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16,
                                                 voff, soff, 0, 0);
    else if constexpr (BYTES == 4)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 4,
                                                 voff, soff, 0, 0);
    else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 2,
                                                 voff, soff, 0, 0);
}

/* Non-temporal 16-byte buffer load (buffer_load_dwordx4 ... nt) at byte `off` of the
 * resource; an offset past the resource's num_records returns zeros without touching
 * memory. */
__device__ __forceinline__ r3d_i32x4 r3d_buf_ld16_stream(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(r3d_i32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 2));
}

/* The fp8 operand of one 128-wide K step for the row starting at p: bytes [16kb, +16)
 * and [64+16kb, +16). */
__device__ __forceinline__ r3d_i32x8 r3d_ld_fp8_operand(const uint8_t* p, int kb) {
    const r3d_i32x4 lo = r3d_ld16(p + 16 * kb);
    const r3d_i32x4 hi = r3d_ld16(p + 64 + 16 * kb);
    const r3d_i32x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return v;
}

__device__ __forceinline__ r3d_i32x8 r3d_ld_fp8_operand_stream(const uint8_t* p, int kb) {
    const r3d_i32x4 lo = r3d_ld16_stream(p + 16 * kb);
    const r3d_i32x4 hi = r3d_ld16_stream(p + 64 + 16 * kb);
    const r3d_i32x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return v;
}

/* f32 -> bf16 bits, round to nearest even; NaN stays a quiet NaN with its sign. */
__device__ __forceinline__ uint16_t r3d_bf16_rne(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

/* Two f32 -> packed bf16 (a in the low half) with one v_cvt_pk_bf16_f32.  On MI355X this
 * is bit-identical to r3d_bf16_rne for every one of the 2^32 f32 inputs (NaN payloads and
 * subnormals included; checked exhaustively on the device). */
__device__ __forceinline__ uint32_t r3d_pack_bf16x2(float a, float b) {
    typedef __bf16 r3d_bf16x2 __attribute__((ext_vector_type(2)));
    typedef float r3d_f32x2 __attribute__((ext_vector_type(2)));
    const r3d_bf16x2 h = __builtin_convertvector(r3d_f32x2{a, b}, r3d_bf16x2);
    return __builtin_bit_cast(uint32_t, h);
}

__device__ __forceinline__ float r3d_bf16_to_f32(uint16_t h) {
    return __uint_as_float((uint32_t)h << 16);
}

#endif /* R3D_DEVICE_H */
