// Device-side helpers shared by the gfx950 kernels of libsf_hip_kernels.so.
//
// Vector types match the operand types of the CDNA4 MFMA builtins.  fp32 ->
// bf16 conversions use gfx950's v_cvt_pk_bf16_f32 (round to nearest even,
// NaN stays NaN), which host tests restate as the usual bit manipulation.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sfk {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
    return __uint_as_float(h << 16);
}

// Two fp32 -> packed bf16x2 (low half = a), one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2v{a, b}, bf16x2v));
}

// fp32 -> bf16 bits, round to nearest even; NaN stays NaN.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}

__device__ __forceinline__ bf16x8 u32x4_as_bf16x8(u32x4 v) {
    return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ bf16x8 load_bf16x8(const uint16_t* p) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(p));
}

__device__ __forceinline__ bf16x8 zero_bf16x8() {
    u32x4 z = {0u, 0u, 0u, 0u};
    return __builtin_bit_cast(bf16x8, z);
}

// D = A(16x32) * B(32x16) + C, fp32 accumulate.  Lane l supplies row l%16
// of A and column l%16 of B, 8 consecutive k values each (group l/16);
// D lane l holds rows 4*(l/16)+i, column l%16.
__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f16x8 u32x4_as_f16x8(u32x4 v) {
    return __builtin_bit_cast(f16x8, v);
}

// Two fp32 -> packed fp16x2 (low half = a), round to nearest even (values
// beyond the fp16 range give +-inf): one v_cvt_pk_f16_f32.
typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_f16x2_rn(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2v{a, b}, f16x2v));
}

// The fp16 form of mfma16x16x32, same operand layout.
__device__ __forceinline__ f32x4 mfma16x16x32_f16(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Raw buffer resource over [base, base + bytes): loads past `bytes` return 0.
// Word 3 = 0x00020000 is the raw-buffer format for the gfx9 family (gfx950).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
}

__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0);
}

// Sum over the 16 lanes of each row (DPP quad permutes, then the row's half
// mirror and mirror: VALU only, no LDS round trip); every lane of the row
// gets the sum, added in the order of an xor butterfly over 1, 2, 4, 8.
__device__ __forceinline__ float row16_sum(float x) {
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, true));   // quad_perm 1,0,3,2
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, true));   // quad_perm 2,3,0,1
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x141, 0xF, 0xF, true));  // row_half_mirror
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x140, 0xF, 0xF, true));  // row_mirror
    return x;
}

// Deferred RMSNorm: the row scale rsqrt(ss / n + eps) from a row's sum of
// squares, and the affine step a consumer applies to its contraction v of
// x * gamma rows: (v * weight scale) * row scale + bias, one rounding for
// the product and one fused multiply-add, the same in every kernel that
// finishes such a projection (so their results agree bit for bit).
__device__ __forceinline__ float deferred_rsqrt(float ss, float inv_n, float eps) {
    return 1.f / sqrtf(ss * inv_n + eps);
}
__device__ __forceinline__ float deferred_affine(float v, float wscale, float rs, float bias) {
    return __builtin_fmaf(v * wscale, rs, bias);
}

__device__ __forceinline__ float fast_exp2(float x) {
    return __builtin_amdgcn_exp2f(x);
}

}  // namespace sfk
