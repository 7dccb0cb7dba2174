// Element-wise kernels of the RDT-1B denoise step (rdt1b.cpp:254-369) and
// the Euler sampler (flow_matching.cpp:69-79), plus device-side synthetic
// weight initialisation.  Each one replaces a chain of reference launches:
//   build_action_input   cast(x_t) + fill(mask, 1) + cat (rdt1b.cpp:286-300)
//   assemble_tokens      expand_to_batch + cat + add(x_pos_embed) (:319-340)
//   add_pos_bf16         add(lang_cond, lang_pos[:L]) / add(img, img_pos) (:342-349)
//   euler_update         slice last T rows + copy + scale(dt) + add
//                        (rdt1b.cpp:362-368, flow_matching.cpp:77-78)
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <math.h>
#include <stdint.h>

#include "sf_device.h"
#include "sf_hip.h"
#include "sf_rdt.h"

namespace sfk {

// Counter-based normal variates: SplitMix64 finaliser of (seed, index) ->
// two uniforms -> Box-Muller.  Element i is a pure function of (seed, i).
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ float normal_at(uint64_t seed, uint64_t i) {
    const uint64_t a = mix64(seed + 0x9E3779B97F4A7C15ull * (2 * i + 1));
    const uint64_t b = mix64(seed + 0x9E3779B97F4A7C15ull * (2 * i + 2));
    const float u1 = ((float)(a >> 40) + 1.f) * (1.f / 16777216.f);   // (0, 1]
    const float u2 = (float)(b >> 40) * (1.f / 16777216.f);           // [0, 1)
    return sqrtf(-2.f * logf(u1)) * cosf(6.2831853071795864f * u2);
}

__global__ void init_normal_kernel(void* p, int bf16, int64_t n, uint64_t seed, float std) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const float v = normal_at(seed, (uint64_t)i) * std;
        if (bf16) reinterpret_cast<uint16_t*>(p)[i] = (uint16_t)f32_to_bf16_bits(v);
        else reinterpret_cast<float*>(p)[i] = v;
    }
}

__global__ void fill_f32_kernel(float* p, int64_t n, float v) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

// Per-row symmetric int8: s = max|w| / 127, q = clamp(rint(w / s), -127, 127);
// w is the row's N(0, std) draw in fp32.  One workgroup of 256 per row.
__global__ __launch_bounds__(256) void quantize_rows_kernel(int8_t* q, float* scale, int64_t K,
                                                            uint64_t seed, float std) {
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    float amax = 0.f;
    for (int64_t c = threadIdx.x; c < K; c += 256)
        amax = fmaxf(amax, fabsf(normal_at(seed, (uint64_t)(row * K + c)) * std));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float s = amax > 0.f ? amax / 127.f : 1.f;
    if (threadIdx.x == 0) scale[row] = s;
    for (int64_t c = threadIdx.x; c < K; c += 256) {
        float v = rintf(normal_at(seed, (uint64_t)(row * K + c)) * std / s);
        v = fminf(127.f, fmaxf(-127.f, v));
        q[row * K + c] = (int8_t)v;
    }
}

__global__ void build_action_input_kernel(const float* x_t, uint16_t* out, int64_t rows, int A) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * 2 * A) return;
    const int64_t r = i / (2 * A);
    const int c = (int)(i % (2 * A));
    const float v = c < A ? x_t[r * A + c] : 1.f;
    out[i] = (uint16_t)f32_to_bf16_bits(v);
}

__global__ void assemble_tokens_kernel(float* x, const float* t_emb, const float* f_emb,
                                       const uint16_t* state, const float* act, const float* pos,
                                       int B, int T, int D) {
    const int S = T + 3;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)B * S * D) return;
    const int d = (int)(i % D);
    const int64_t row = i / D;
    const int b = (int)(row / S);
    const int s = (int)(row % S);
    float v;
    if (s == 0) v = t_emb[d];
    else if (s == 1) v = f_emb[d];
    else if (s == 2) v = bf16_bits_to_f32(state[(int64_t)b * D + d]);
    else v = act[((int64_t)b * T + (s - 3)) * D + d];
    x[i] = v + pos[(int64_t)s * D + d];
}

__global__ void add_pos_bf16_kernel(const uint16_t* tok, const float* pos, uint16_t* out, int B,
                                    int L, int D) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)B * L * D) return;
    const int64_t ld = i % ((int64_t)L * D);
    out[i] = (uint16_t)f32_to_bf16_bits(bf16_bits_to_f32(tok[i]) + pos[ld]);
}

__global__ void euler_update_kernel(float* x, const float* v, int B, int T, int A, int S,
                                    float dt) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)B * T * A) return;
    const int a = (int)(i % A);
    const int64_t bt = i / A;
    const int b = (int)(bt / T);
    const int t = (int)(bt % T);
    const float step = dt * v[((int64_t)b * S + 3 + t) * A + a];
    x[i] = x[i] + step;
}

inline unsigned blocks_for(int64_t n, int per = 256) {
    int64_t b = (n + per - 1) / per;
    return (unsigned)(b > 0x7fffffff ? 0x7fffffff : b);
}

// Largest |x| over n bf16 values, merged into *out (fp32 bits, so the
// integer maximum of non-negative values is their float maximum; NaN bit
// patterns order above inf, so a NaN anywhere gives a NaN result).  Eight
// values (16 bytes) per thread and step; the workgroup's maximum goes out
// as one atomic (all workgroups target the same word, so there are few).
__global__ __launch_bounds__(256) void absmax_bf16_kernel(const uint16_t* __restrict__ p, int64_t n,
                                                          unsigned int* out) {
    uint32_t m = 0;
    const int64_t n8 = n / 8;
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += stride) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(p + 8 * i);
#pragma unroll
        for (int e = 0; e < 4; ++e) m = max(m, max(w[e] & 0x7fffu, (w[e] >> 16) & 0x7fffu));
    }
    for (int64_t i = 8 * n8 + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
        m = max(m, (uint32_t)(p[i] & 0x7fffu));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, off, 64));
    __shared__ uint32_t wm[4];
    if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        m = max(max(wm[0], wm[1]), max(wm[2], wm[3]));
        if (m) atomicMax(out, m << 16);
    }
}

// absmax_bf16_kernel over up to SF_ABSMAX_MAX_JOBS buffers in one launch:
// workgroup row blockIdx.y takes buffer j (its own output word), the x
// extent strides over it.
struct AbsmaxJobs {
    const uint16_t* p[SF_ABSMAX_MAX_JOBS];
    int64_t n[SF_ABSMAX_MAX_JOBS];
    unsigned int* out[SF_ABSMAX_MAX_JOBS];
};

__global__ __launch_bounds__(256) void absmax_jobs_kernel(const AbsmaxJobs J) {
    const int j = blockIdx.y;
    const uint16_t* __restrict__ p = J.p[j];
    const int64_t n = J.n[j];
    uint32_t m = 0;
    const int64_t n8 = n / 8;
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += stride) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(p + 8 * i);
#pragma unroll
        for (int e = 0; e < 4; ++e) m = max(m, max(w[e] & 0x7fffu, (w[e] >> 16) & 0x7fffu));
    }
    for (int64_t i = 8 * n8 + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
        m = max(m, (uint32_t)(p[i] & 0x7fffu));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, off, 64));
    __shared__ uint32_t wm[4];
    if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        m = max(max(wm[0], wm[1]), max(wm[2], wm[3]));
        if (m) atomicMax(J.out[j], m << 16);
    }
}

// In place bf16 -> fp16 (nearest even) of buffer blockIdx.y when the max |x|
// absmax_jobs_kernel merged for it is below `limit` (a NaN maximum is not):
// the same conversion the attention's fp16 P.V form applies to bf16 V in
// registers (pack_f16x2_rn of each element's fp32 value), done once.
// The maximum is compared as bits: a non-negative float orders like its bit
// pattern and every NaN pattern lies above +inf, so this holds whatever the
// compiler assumes about NaN (the library is built with -fno-honor-nans,
// under which !(mx < limit) may become mx >= limit).  limit > 0.
__global__ __launch_bounds__(256) void to_f16_below_kernel(const AbsmaxJobs J, uint32_t limit_bits) {
    const int j = blockIdx.y;
    if (*J.out[j] >= limit_bits) return;
    uint16_t* __restrict__ p = const_cast<uint16_t*>(J.p[j]);
    const int64_t n = J.n[j];
    const int64_t n8 = n / 8;
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += stride) {
        u32x4 w = *reinterpret_cast<const u32x4*>(p + 8 * i);
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = pack_f16x2_rn(__uint_as_float(w[e] << 16), __uint_as_float(w[e] & 0xffff0000u));
        *reinterpret_cast<u32x4*>(p + 8 * i) = w;
    }
    for (int64_t i = 8 * n8 + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
        p[i] = (uint16_t)(pack_f16x2_rn(__uint_as_float((uint32_t)p[i] << 16), 0.f) & 0xffffu);
}

}  // namespace sfk

using sfk::blocks_for;

extern "C" int sf_init_normal(void* p, int32_t dtype, int64_t n, uint64_t seed, float std,
                              void* stream) {
    if (n < 0 || (n && !p)) return SF_EINVAL;
    if (dtype != SF_BF16 && dtype != SF_F32) return SF_ENOTSUP;
    if (!n) return SF_OK;
    const unsigned g = blocks_for(n) < 16384 ? blocks_for(n) : 16384;
    hipLaunchKernelGGL(sfk::init_normal_kernel, dim3(g), dim3(256), 0,
                       static_cast<hipStream_t>(stream), p, dtype == SF_BF16, n, seed, std);
    return hipGetLastError() == hipSuccess ? SF_OK : SF_ELAUNCH;
}

extern "C" int sf_fill_f32(float* p, int64_t n, float v, void* stream) {
    if (n < 0 || (n && !p)) return SF_EINVAL;
    if (!n) return SF_OK;
    const unsigned g = blocks_for(n) < 16384 ? blocks_for(n) : 16384;
    hipLaunchKernelGGL(sfk::fill_f32_kernel, dim3(g), dim3(256), 0, static_cast<hipStream_t>(stream),
                       p, n, v);
    return hipGetLastError() == hipSuccess ? SF_OK : SF_ELAUNCH;
}

extern "C" int sf_init_int8_rows(int8_t* q, float* scale, int64_t N, int64_t K, uint64_t seed,
                                 float std, void* stream) {
    if (N < 0 || K <= 0 || (N && (!q || !scale))) return SF_EINVAL;
    if (!N) return SF_OK;
    hipLaunchKernelGGL(sfk::quantize_rows_kernel, dim3((unsigned)N), dim3(256), 0,
                       static_cast<hipStream_t>(stream), q, scale, K, seed, std);
    return hipGetLastError() == hipSuccess ? SF_OK : SF_ELAUNCH;
}

extern "C" int sf_build_action_input(const float* x_t, void* out, int64_t rows, int32_t A,
                                     void* stream) {
    if (!x_t || !out || rows < 0 || A <= 0) return SF_EINVAL;
    if (!rows) return SF_OK;
    hipLaunchKernelGGL(sfk::build_action_input_kernel, dim3(blocks_for(rows * 2 * A)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), x_t, static_cast<uint16_t*>(out), rows, A);
    return hipGetLastError() == hipSuccess ? SF_OK : SF_ELAUNCH;
}

extern "C" int sf_assemble_tokens(float* x, const float* t_emb, const float* f_emb,
                                  const void* state, const float* act, const float* pos, int32_t B,
                                  int32_t T, int32_t D, void* stream) {
    if (!x || !t_emb || !f_emb || !state || !act || !pos || B < 0 || T < 0 || D <= 0)
        return SF_EINVAL;
    const int64_t n = (int64_t)B * (T + 3) * D;
    if (!n) return SF_OK;
    hipLaunchKernelGGL(sfk::assemble_tokens_kernel, dim3(blocks_for(n)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), x, t_emb, f_emb,
                       static_cast<const uint16_t*>(state), act, pos, B, T, D);
    return hipGetLastError() == hipSuccess ? SF_OK : SF_ELAUNCH;
}

extern "C" int sf_add_pos_bf16(const void* tok, const float* pos, void* out, int32_t B, int32_t L,
                               int32_t D, void* stream) {
    if (!tok || !pos || !out || B < 0 || L < 0 || D <= 0) return SF_EINVAL;
    const int64_t n = (int64_t)B * L * D;
    if (!n) return SF_OK;
    hipLaunchKernelGGL(sfk::add_pos_bf16_kernel, dim3(blocks_for(n)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(tok), pos,
                       static_cast<uint16_t*>(out), B, L, D);
    return hipGetLastError() == hipSuccess ? SF_OK : SF_ELAUNCH;
}

extern "C" int sf_euler_update(float* x, const float* v, int32_t B, int32_t T, int32_t A,
                               int32_t S, float dt, void* stream) {
    if (!x || !v || B < 0 || T < 0 || A <= 0 || S < T + 3) return SF_EINVAL;
    const int64_t n = (int64_t)B * T * A;
    if (!n) return SF_OK;
    hipLaunchKernelGGL(sfk::euler_update_kernel, dim3(blocks_for(n)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), x, v, B, T, A, S, dt);
    return hipGetLastError() == hipSuccess ? SF_OK : SF_ELAUNCH;
}

extern "C" int sf_absmax_bf16_batched(const sf_absmax_job* jobs, int32_t count, void* stream) {
    if (count < 0 || count > SF_ABSMAX_MAX_JOBS || (count && !jobs)) return SF_EINVAL;
    sfk::AbsmaxJobs J{};
    int64_t most = 0;
    for (int j = 0; j < count; ++j) {
        const sf_absmax_job& b = jobs[j];
        if (!b.out || b.n < 0 || (b.n && !b.p) || (reinterpret_cast<uintptr_t>(b.p) & 15)) return SF_EINVAL;
        J.p[j] = static_cast<const uint16_t*>(b.p);
        J.n[j] = b.n;
        J.out[j] = reinterpret_cast<unsigned int*>(b.out);
        most = std::max(most, b.n);
    }
    if (!count || !most) return SF_OK;
    const int64_t want = (most / 8 + 255) / 256;
    const unsigned blocks = (unsigned)std::max<int64_t>(1, std::min<int64_t>(want, 256));
    hipLaunchKernelGGL(sfk::absmax_jobs_kernel, dim3(blocks, (unsigned)count), dim3(256), 0,
                       static_cast<hipStream_t>(stream), J);
    return hipGetLastError() == hipSuccess ? SF_OK : SF_ELAUNCH;
}

extern "C" int sf_bf16_to_f16_below(const sf_absmax_job* jobs, int32_t count, float limit, void* stream) {
    if (count < 0 || count > SF_ABSMAX_MAX_JOBS || (count && !jobs)) return SF_EINVAL;
    if (!(limit > 0.f)) return SF_EINVAL;
    sfk::AbsmaxJobs J{};
    int64_t most = 0;
    for (int j = 0; j < count; ++j) {
        const sf_absmax_job& b = jobs[j];
        if (!b.out || b.n < 0 || (b.n && !b.p) || (reinterpret_cast<uintptr_t>(b.p) & 15)) return SF_EINVAL;
        J.p[j] = static_cast<const uint16_t*>(b.p);
        J.n[j] = b.n;
        J.out[j] = reinterpret_cast<unsigned int*>(b.out);
        most = std::max(most, b.n);
    }
    if (!count || !most) return SF_OK;
    const int64_t want = (most / 8 + 255) / 256;
    const unsigned blocks = (unsigned)std::max<int64_t>(1, std::min<int64_t>(want, 1024));
    uint32_t limit_bits;
    std::memcpy(&limit_bits, &limit, 4);
    hipLaunchKernelGGL(sfk::to_f16_below_kernel, dim3(blocks, (unsigned)count), dim3(256), 0,
                       static_cast<hipStream_t>(stream), J, limit_bits);
    return hipGetLastError() == hipSuccess ? SF_OK : SF_ELAUNCH;
}

extern "C" int sf_absmax_bf16(const void* p, int64_t n, float* out, void* stream) {
    if (!p || !out || n < 0) return SF_EINVAL;
    if (reinterpret_cast<uintptr_t>(p) & 15) return SF_EINVAL;
    if (!n) return SF_OK;
    const int64_t want = (n / 8 + 255) / 256;
    const unsigned blocks = (unsigned)std::max<int64_t>(1, std::min<int64_t>(want, 256));
    hipLaunchKernelGGL(sfk::absmax_bf16_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint16_t*>(p), n, reinterpret_cast<unsigned int*>(out));
    return hipGetLastError() == hipSuccess ? SF_OK : SF_ELAUNCH;
}
