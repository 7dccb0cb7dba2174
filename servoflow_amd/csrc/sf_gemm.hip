// Projection GEMMs of the RDT-1B block on MI355X (gfx950).
//
// Replaces gemm_bias_act (src/backend/cuda/cuda_backend.cu:337-467, the
// cuBLASLt BIAS / GELU_BIAS epilogues, SiLU applied after at :449-451) as the
// RDT layers call it: C[M,N] = act(A[M,K] . W[N,K]^T + bias[N])
// (trans_b = true, dit_block.cu:207, 233, 284, 291, 321, 152-160), plus the
// neighbouring ops folded into the epilogue:
//   * residual add (the x += branch adds of dit_block.cu:372, 379, 384),
//   * split into per-head [B,H,S,D] tensors with the per-head RMSNorm of
//     q_norm / k_norm (split_qkv, split_kv, seq_to_head of
//     src/backend/cuda/ops/split_ops.cuh:62-84, 123-137, 210-226 followed by
//     rms_norm_kernel_impl, norm.cuh:89-122, over head_dim),
//   * int8 weight-only dequantisation (dequantize_int8_fp16_kernel,
//     src/backend/cuda/ops/quantization.cu:18-51): int8 codes are widened to
//     bf16 exactly in registers and the per-row fp32 scale multiplies the dot
//     product in the epilogue (sum_k (q_nk s_n) a_mk = s_n sum_k q_nk a_mk).
//
// Shape regime: at batch 1 the RDT projections have M = 67 rows, so every
// GEMM is weight streaming (arithmetic intensity = M flop/byte).  The kernel
// computes C^T = W . A^T so weight rows are MFMA rows: each lane loads 16
// contiguous bytes of a weight row straight from HBM into the operand
// registers (no LDS staging, every weight byte is read once), and the few
// activation rows are the MFMA columns, read from L2.  A workgroup of 8
// waves covers NR weight rows over all of K: the waves split K and reduce
// in LDS, so no split-K partials touch HBM.  M > 80 is handled as a grid of
// 80-row tiles.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <algorithm>

#include "sf_device.h"
#include "sf_hip.h"

namespace sfk {

constexpr int kGemmThreads = 512;   // 8 waves

struct GemmArgs {
    const uint16_t* a;     // [M][lda] bf16
    const void* w;         // [N][ldw] bf16 or int8
    const float* w_scale;  // [N] (int8 weights)
    const float* bias;     // [N] or null
    void* c;               // [M][ldc] bf16 / f32
    int64_t lda, ldw, ldc;
    int M, N, K;
    int act;               // 0 none, 1 GELU(tanh), 2 SiLU
    int c_f32;
    int accumulate;        // c (f32) += result
    // per-head epilogue
    int heads;             // 1: columns are sections of H*64 -> [B,H,S,D]
    int H, S;
    float eps;
    const float* head_gamma[3];
    uint16_t* head_out[3];
    int64_t head_sb[3], head_sh[3], head_ss[3];
};

__device__ __forceinline__ float gelu_tanh(float x) {
    // GeluOp, src/backend/cuda/ops/elementwise.cuh:35-54.
    const float kAlpha = 0.7978845608028654f;
    const float kBeta = 0.044715f;
    return 0.5f * x * (1.f + tanhf(kAlpha * (x + kBeta * x * x * x)));
}

__device__ __forceinline__ float silu(float x) { return x / (1.f + expf(-x)); }

__device__ __forceinline__ float apply_act(int act, float v) {
    return act == 1 ? gelu_tanh(v) : (act == 2 ? silu(v) : v);
}

// Eight int8 codes -> bf16x8 (exact: |code| <= 128 needs 8 significant bits).
__device__ __forceinline__ bf16x8 i8x8_to_bf16x8(uint2 raw) {
    uint32_t w[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const uint32_t src = p < 2 ? raw.x : raw.y;
        const int sh = (p & 1) * 16;
        const float lo = (float)(int)(int8_t)(src >> sh);
        const float hi = (float)(int)(int8_t)(src >> (sh + 8));
        w[p] = __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
    }
    return u32x4_as_bf16x8(u32x4{w[0], w[1], w[2], w[3]});
}

// NR weight rows per workgroup: 16 (plain epilogue, K split 8 ways) or 64
// (one attention head, K split 2 ways, per-head epilogue).  MB activation
// blocks of 16 rows.  W8: int8 weights.
template <int NR, int MB, bool W8>
__global__ __launch_bounds__(kGemmThreads) void gemm_smallm_kernel(const GemmArgs g) {
    constexpr int KS = 8 / (NR / 16);         // waves sharing one n-block
    constexpr int MR = 16 * MB;
    __shared__ __attribute__((aligned(16))) float red[KS * NR * MR];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int g4 = lane >> 4;
    const int r = lane & 15;
    const int nb = w % (NR / 16);
    const int ks = w / (NR / 16);
    const int nrow0 = blockIdx.x * NR;
    const int m0 = blockIdx.y * MR;

    // K slice of this wave, in 32-wide chunks.
    const int nchunks = g.K / 32;
    const int per = (nchunks + KS - 1) / KS;
    const int c_beg = ks * per;
    const int c_end = min(nchunks, c_beg + per);

    const int wrow = nrow0 + 16 * nb + r;
    const int wbytes = W8 ? 1 : 2;
    const __amdgpu_buffer_rsrc_t wrs =
        make_rsrc(g.w, (uint32_t)min((int64_t)g.N * g.ldw * wbytes, (int64_t)0x7fffffff));
    const __amdgpu_buffer_rsrc_t ars = make_rsrc(g.a + (int64_t)m0 * g.lda,
                                                 (uint32_t)((int64_t)max(0, min(MR, g.M - m0)) * g.lda * 2));
    // Rows past N (and activation rows past M) read as zeros.
    const uint32_t wrow_off = wrow < g.N ? (uint32_t)((int64_t)wrow * g.ldw * wbytes) : 0x80000000u;

    f32x4 acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};

    constexpr int U = 8;   // chunks in flight per wave
    for (int c0 = c_beg; c0 < c_end; c0 += U) {
        bf16x8 wv[U];
        bf16x8 av[U][MB];
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const int c = c0 + j;
            const bool live = c < c_end;
            const int k = 32 * c + 8 * g4;
            if constexpr (W8) {
                const uint32_t off = live ? wrow_off + (uint32_t)k : 0x80000000u;
                const uint2 raw = __builtin_bit_cast(
                    uint2, __builtin_amdgcn_raw_buffer_load_b64(wrs, off, 0, 0));
                wv[j] = i8x8_to_bf16x8(raw);
            } else {
                const uint32_t off = live ? wrow_off + (uint32_t)k * 2 : 0x80000000u;
                wv[j] = __builtin_bit_cast(bf16x8, buffer_load16(wrs, off));
            }
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const uint32_t off = live ? (uint32_t)(((16 * mb + r) * g.lda + k) * 2) : 0x80000000u;
                av[j][mb] = __builtin_bit_cast(bf16x8, buffer_load16(ars, off));
            }
        }
#pragma unroll
        for (int j = 0; j < U; ++j) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) acc[mb] = mfma16x16x32(wv[j], av[j][mb], acc[mb]);
        }
    }

    // Partial C^T over this wave's K slice: lane holds n = 16nb + 4g4 + i,
    // m = 16mb + r.  Layout red[ks][n][m].
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            red[(ks * NR + 16 * nb + 4 * g4 + i) * MR + 16 * mb + r] = acc[mb][i];
    }
    __syncthreads();

    if (!g.heads) {
        for (int idx = tid; idx < NR * MR; idx += kGemmThreads) {
            const int nn = idx % NR;
            const int mm = idx / NR;
            const int n = nrow0 + nn;
            const int m = m0 + mm;
            if (n >= g.N || m >= g.M) continue;
            float v = 0.f;
#pragma unroll
            for (int s = 0; s < KS; ++s) v += red[(s * NR + nn) * MR + mm];
            if (W8) v *= g.w_scale[n];
            if (g.bias) v += g.bias[n];
            v = apply_act(g.act, v);
            const int64_t off = (int64_t)m * g.ldc + n;
            if (g.c_f32) {
                float* cp = reinterpret_cast<float*>(g.c) + off;
                *cp = g.accumulate ? *cp + v : v;
            } else {
                reinterpret_cast<uint16_t*>(g.c)[off] = (uint16_t)f32_to_bf16_bits(v);
            }
        }
    } else {
        // One head (64 columns): optional RMSNorm over the head dim, then
        // bf16 store to out[b][h][s][d] with m = b*S + s.
        const int hd_cols = g.H * 64;
        const int sec = nrow0 / hd_cols;
        const int h = (nrow0 % hd_cols) / 64;
        const float* gamma = g.head_gamma[sec];
        uint16_t* outp = g.head_out[sec];
        const int d = lane;
        const int n = nrow0 + d;
        float bscale = W8 ? g.w_scale[n] : 1.f;
        const float bia = g.bias ? g.bias[n] : 0.f;
        for (int mm = w; mm < MR; mm += 8) {
            const int m = m0 + mm;
            if (m >= g.M) break;
            float v = 0.f;
#pragma unroll
            for (int s = 0; s < KS; ++s) v += red[(s * NR + d) * MR + mm];
            v = v * bscale + bia;
            if (gamma) {
                // rms_norm_kernel_impl over the 64 head dims (norm.cuh:89-122)
                float ss = v * v;
#pragma unroll
                for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
                const float inv_rms = 1.f / sqrtf(ss / 64.f + g.eps);
                v = v * inv_rms * gamma[d];
            }
            const int bb = m / g.S;
            const int s = m % g.S;
            outp[bb * g.head_sb[sec] + h * g.head_sh[sec] + s * g.head_ss[sec] + d] =
                (uint16_t)f32_to_bf16_bits(v);
        }
    }
}

template <int NR, bool W8>
hipError_t launch_smallm(const GemmArgs& g, int mb, dim3 grid, hipStream_t s) {
    switch (mb) {
        case 1: hipLaunchKernelGGL((gemm_smallm_kernel<NR, 1, W8>), grid, dim3(kGemmThreads), 0, s, g); break;
        case 2: hipLaunchKernelGGL((gemm_smallm_kernel<NR, 2, W8>), grid, dim3(kGemmThreads), 0, s, g); break;
        case 3: hipLaunchKernelGGL((gemm_smallm_kernel<NR, 3, W8>), grid, dim3(kGemmThreads), 0, s, g); break;
        case 4: hipLaunchKernelGGL((gemm_smallm_kernel<NR, 4, W8>), grid, dim3(kGemmThreads), 0, s, g); break;
        default: hipLaunchKernelGGL((gemm_smallm_kernel<NR, 5, W8>), grid, dim3(kGemmThreads), 0, s, g); break;
    }
    return hipGetLastError();
}

}  // namespace sfk

// ---------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------
namespace {
bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
}  // namespace

extern "C" int sf_gemm(const sf_gemm_desc* d, void* stream) {
    if (!d) return SF_EINVAL;
    if (d->M < 0 || d->N < 0 || d->K < 0) return SF_EINVAL;
    if ((long)d->M * d->N == 0) return SF_OK;
    if (d->K == 0 || (d->K & 31)) return SF_ENOTSUP;
    if (d->a_dtype != SF_BF16) return SF_ENOTSUP;
    if (d->w_dtype != SF_BF16 && d->w_dtype != SF_I8) return SF_ENOTSUP;
    if (d->act < 0 || d->act > 2) return SF_EINVAL;
    if (!d->A || !d->W) return SF_EINVAL;
    if (!al16(d->A) || !al16(d->W) || (d->lda & 7) || d->lda < d->K) return SF_EINVAL;
    if (d->w_dtype == SF_BF16 && ((d->ldw & 7) || d->ldw < d->K)) return SF_EINVAL;
    if (d->w_dtype == SF_I8 && ((d->ldw & 7) || d->ldw < d->K || !d->w_scale)) return SF_EINVAL;
    if ((int64_t)std::max(1, std::min(80, d->M)) * d->lda * 2 > 0x7fffffffLL) return SF_ENOTSUP;
    sfk::GemmArgs g{};
    g.a = static_cast<const uint16_t*>(d->A);
    g.w = d->W;
    g.w_scale = d->w_scale;
    g.bias = d->bias;
    g.lda = d->lda;
    g.ldw = d->ldw;
    g.M = d->M; g.N = d->N; g.K = d->K;
    g.act = d->act;
    g.eps = d->eps;
    const bool w8 = d->w_dtype == SF_I8;
    if (d->epilogue == SF_EPI_HEADS) {
        if (d->H <= 0 || d->S <= 0 || d->M % d->S) return SF_EINVAL;
        const int cols = d->H * 64;
        if (d->N % cols || d->N / cols > 3) return SF_EINVAL;
        for (int j = 0; j < d->N / cols; ++j) {
            if (!d->head_out[j]) return SF_EINVAL;
            g.head_out[j] = static_cast<uint16_t*>(d->head_out[j]);
            g.head_gamma[j] = d->head_gamma[j];
            g.head_sb[j] = d->head_stride[j][0];
            g.head_sh[j] = d->head_stride[j][1];
            g.head_ss[j] = d->head_stride[j][2];
        }
        g.heads = 1;
        g.H = d->H;
        g.S = d->S;
    } else if (d->epilogue == SF_EPI_PLAIN) {
        if (!d->C || d->ldc < d->N) return SF_EINVAL;
        if (d->c_dtype != SF_BF16 && d->c_dtype != SF_F32) return SF_ENOTSUP;
        if (d->accumulate && d->c_dtype != SF_F32) return SF_EINVAL;
        g.c = d->C;
        g.ldc = d->ldc;
        g.c_f32 = d->c_dtype == SF_F32;
        g.accumulate = d->accumulate != 0;
    } else {
        return SF_EINVAL;
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int mtiles = (d->M + 79) / 80;
    const int mb = d->M >= 80 ? 5 : (d->M + 15) / 16;
    hipError_t e;
    if (g.heads) {
        const dim3 grid(d->N / 64, mtiles);
        e = w8 ? sfk::launch_smallm<64, true>(g, mb, grid, s) : sfk::launch_smallm<64, false>(g, mb, grid, s);
    } else {
        const dim3 grid((d->N + 15) / 16, mtiles);
        e = w8 ? sfk::launch_smallm<16, true>(g, mb, grid, s) : sfk::launch_smallm<16, false>(g, mb, grid, s);
    }
    return e == hipSuccess ? SF_OK : SF_ELAUNCH;
}
