// Row normalisation and int8 dequant for the RDT-1B block on MI355X.
//
// rmsnorm / add_rmsnorm replace rms_norm_kernel_impl and
// fused_add_rms_norm_kernel (src/backend/cuda/ops/norm.cuh:89-122, 130-171):
// one workgroup of 256 threads per row, 16-byte vector loads, fp32 sums
// reduced with cross-lane shuffles and one LDS step (the reference reduces a
// 256-entry LDS array with a barrier per halving).  The residual stays fp32.
// dequant replaces dequantize_int8_fp16_kernel (quantization.cu:18-51).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "sf_device.h"
#include "sf_hip.h"

namespace sfk {

constexpr int kNormThreads = 256;

__device__ __forceinline__ float block_sum_256(float v, float* red) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

__device__ __forceinline__ float load_elem(const void* p, int bf16, int64_t i) {
    return bf16 ? bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i])
                : reinterpret_cast<const float*>(p)[i];
}

// kind: 0 fp32, 1 bf16, 2 fp16
__device__ __forceinline__ void store_elem(void* p, int kind, int64_t i, float v) {
    if (kind == 1) reinterpret_cast<uint16_t*>(p)[i] = (uint16_t)f32_to_bf16_bits(v);
    else if (kind == 2) reinterpret_cast<_Float16*>(p)[i] = (_Float16)v;
    else reinterpret_cast<float*>(p)[i] = v;
}

int out_kind(int32_t dtype) { return dtype == SF_BF16 ? 1 : (dtype == SF_F16 ? 2 : 0); }

// Each thread owns up to kPer columns of its row in registers.
constexpr int kPer = 16;   // 256 threads x 16 = 4096 columns max per row

__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(
    const void* x, int x_bf16, int64_t ldx, const void* delta, int delta_bf16, float* residual,
    const float* gamma, void* out, int okind, int64_t ldo, int cols, float eps) {
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    float v[kPer];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int c = threadIdx.x + kNormThreads * j;
        float e = 0.f;
        if (c < cols) {
            if (residual) {
                e = residual[row * cols + c] + load_elem(delta, delta_bf16, row * cols + c);
                residual[row * cols + c] = e;
            } else {
                e = load_elem(x, x_bf16, row * ldx + c);
            }
        }
        v[j] = e;
        ss += e * e;
    }
    const float total = block_sum_256(ss, red);
    const float inv_rms = 1.f / sqrtf(total / (float)cols + eps);
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int c = threadIdx.x + kNormThreads * j;
        if (c < cols) store_elem(out, okind, row * ldo + c, v[j] * inv_rms * gamma[c]);
    }
}

// Deferred form (no normalisation yet): out = x * gamma and ss[t][row] =
// the sum of x^2 over the 64 columns of tile t, one workgroup per 16 rows x
// 64 columns (lanes 16k .. 16k + 15 share a row, 4 columns each); the same
// layout and summation order as the GEMM's deferred residual add + norm.
__global__ __launch_bounds__(256) void norm_deferred_kernel(const float* x, int64_t ldx, const float* gamma,
                                                            void* out, int okind, int64_t ldo, float* ss,
                                                            int rows, int cols) {
    const int ntl = cols / 64;
    const int r = (int)(blockIdx.x / ntl) * 16 + (int)(threadIdx.x >> 4);
    const int c = 64 * (int)(blockIdx.x % ntl) + 4 * (int)(threadIdx.x & 15);
    if (r >= rows) return;   // whole 16-lane groups
    const f32x4 v = *reinterpret_cast<const f32x4*>(x + (int64_t)r * ldx + c);
    const f32x4 g = *reinterpret_cast<const f32x4*>(gamma + c);
#pragma unroll
    for (int j = 0; j < 4; ++j) store_elem(out, okind, (int64_t)r * ldo + c + j, v[j] * g[j]);
    const float t = row16_sum(v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3]);
    if ((threadIdx.x & 15) == 0) ss[(int64_t)(c / 64) * rows + r] = t;
}

__global__ __launch_bounds__(256) void dequant_int8_kernel(const int8_t* q, const float* scale,
                                                           int per_channel, void* out, int out_bf16,
                                                           int64_t n, int64_t K) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float s = per_channel ? scale[i / K] : scale[0];   // row = i / K (quantization.cu:35)
    store_elem(out, out_bf16, i, (float)q[i] * s);
}

}  // namespace sfk

extern "C" int sf_rmsnorm(const void* x, int32_t x_dtype, int64_t ldx, const float* gamma, void* out,
                          int32_t out_dtype, int64_t ldo, int32_t rows, int32_t cols, float eps,
                          void* stream) {
    if (rows < 0 || cols < 0) return SF_EINVAL;
    if ((long)rows * cols == 0) return SF_OK;
    if (!x || !gamma || !out || ldx < cols || ldo < cols) return SF_EINVAL;
    if (x_dtype != SF_F32 && x_dtype != SF_BF16) return SF_ENOTSUP;
    if (out_dtype != SF_F32 && out_dtype != SF_BF16 && out_dtype != SF_F16) return SF_ENOTSUP;
    if (cols > sfk::kNormThreads * sfk::kPer) return SF_ENOTSUP;
    hipLaunchKernelGGL(sfk::rmsnorm_kernel, dim3(rows), dim3(sfk::kNormThreads), 0,
                       static_cast<hipStream_t>(stream), x, x_dtype == SF_BF16, ldx, nullptr, 0,
                       nullptr, gamma, out, sfk::out_kind(out_dtype), ldo, cols, eps);
    return hipGetLastError() == hipSuccess ? SF_OK : SF_ELAUNCH;
}

extern "C" int sf_rmsnorm_deferred(const float* x, int64_t ldx, const float* gamma, void* out, int32_t out_dtype,
                                   int64_t ldo, float* ss, int32_t rows, int32_t cols, void* stream) {
    if (rows < 0 || cols < 0) return SF_EINVAL;
    if ((long)rows * cols == 0) return SF_OK;
    if (!x || !gamma || !out || !ss || ldx < cols || ldo < cols) return SF_EINVAL;
    if (out_dtype != SF_F32 && out_dtype != SF_BF16 && out_dtype != SF_F16) return SF_ENOTSUP;
    if ((cols & 63) || (ldx & 3) || ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(gamma)) & 15))
        return SF_EINVAL;
    const int64_t blocks = (int64_t)(cols / 64) * ((rows + 15) / 16);
    if (blocks > 0x7fffffffLL) return SF_ENOTSUP;
    hipLaunchKernelGGL(sfk::norm_deferred_kernel, dim3((unsigned)blocks), dim3(256), 0,
                       static_cast<hipStream_t>(stream), x, ldx, gamma, out, sfk::out_kind(out_dtype), ldo, ss,
                       rows, cols);
    return hipGetLastError() == hipSuccess ? SF_OK : SF_ELAUNCH;
}

extern "C" int sf_add_rmsnorm(const void* delta, int32_t delta_dtype, float* residual,
                              const float* gamma, void* out, int32_t out_dtype, int32_t rows,
                              int32_t cols, float eps, void* stream) {
    if (rows < 0 || cols < 0) return SF_EINVAL;
    if ((long)rows * cols == 0) return SF_OK;
    if (!delta || !residual || !gamma || !out) return SF_EINVAL;
    if (delta_dtype != SF_F32 && delta_dtype != SF_BF16) return SF_ENOTSUP;
    if (out_dtype != SF_F32 && out_dtype != SF_BF16 && out_dtype != SF_F16) return SF_ENOTSUP;
    if (cols > sfk::kNormThreads * sfk::kPer) return SF_ENOTSUP;
    hipLaunchKernelGGL(sfk::rmsnorm_kernel, dim3(rows), dim3(sfk::kNormThreads), 0,
                       static_cast<hipStream_t>(stream), nullptr, 0, (int64_t)cols, delta,
                       delta_dtype == SF_BF16, residual, gamma, out, sfk::out_kind(out_dtype),
                       (int64_t)cols, cols, eps);
    return hipGetLastError() == hipSuccess ? SF_OK : SF_ELAUNCH;
}

extern "C" int sf_dequant_int8(const int8_t* q, const float* scale, int32_t per_channel, void* out,
                               int32_t out_dtype, int64_t N, int64_t K, void* stream) {
    if (N < 0 || K < 0) return SF_EINVAL;
    const int64_t n = N * K;
    if (n == 0) return SF_OK;
    if (!q || !scale || !out) return SF_EINVAL;
    if (out_dtype != SF_F32 && out_dtype != SF_BF16) return SF_ENOTSUP;
    const int64_t blocks = (n + 255) / 256;
    if (blocks > 0x7fffffffLL) return SF_ENOTSUP;
    hipLaunchKernelGGL(sfk::dequant_int8_kernel, dim3((unsigned)blocks), dim3(256), 0,
                       static_cast<hipStream_t>(stream), q, scale, per_channel != 0, out,
                       out_dtype == SF_BF16, n, K);
    return hipGetLastError() == hipSuccess ? SF_OK : SF_ELAUNCH;
}
