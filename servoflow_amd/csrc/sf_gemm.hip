// Projection GEMMs of the RDT-1B block on MI355X (gfx950).
//
// Replaces gemm_bias_act (src/backend/cuda/cuda_backend.cu:337-467, the
// cuBLASLt BIAS / GELU_BIAS epilogues, SiLU applied after at :449-451) as the
// RDT layers call it: C[M,N] = act(A[M,K] . W[N,K]^T + bias[N])
// (trans_b = true, dit_block.cu:207, 233, 284, 291, 321, 152-160), plus the
// neighbouring ops folded into the epilogue:
//   * residual add (the x += branch adds of dit_block.cu:372, 379, 384) and
//     the RMSNorm that follows it (fused_add_rms_norm_kernel,
//     src/backend/cuda/ops/norm.cuh:130-171, as norm2 / norm3 / next norm1),
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
// GEMM is weight streaming (arithmetic intensity = M flop/byte).  Both paths
// compute C^T = W . A^T so weight rows are MFMA rows: each lane loads 16
// contiguous bytes of a weight row straight from HBM into the operand
// registers (no LDS staging, every weight byte is read once) and the few
// activation rows are the MFMA columns.
//
//   split-K path (M <= 160, caller workspace): a 2048 x 2048 weight is only
//   32 KB per CU, so the matrix is cut into 64-row x KT-wide tiles, one per
//   workgroup, enough to cover all 256 CUs.  Each workgroup issues all of its
//   weight loads at once, stages its activation slice in LDS once for its
//   waves, and writes fp32 partial sums; a reduce kernel sums the K slices in
//   a fixed order (deterministic) and applies the epilogue, including the
//   residual add + RMSNorm that follows a block branch.  That RMSNorm can be
//   deferred (norm_ss): the reduce then runs over 64-column tiles, stores
//   x * gamma and each tile's per-row sum of squares, and the consuming
//   projection (a_row_ss) applies rsqrt(sum / n + eps) to its contraction,
//   since (s a) W^T = s (a W^T) -- no kernel waits for a whole row.
//   library path (M > 160, caller workspace): at those sizes the product is
//   MFMA-bound, a plain library GEMM: hipBLASLt computes it chunk by chunk
//   (<= 8192 rows) and the same epilogue kernels finish it.  What hipBLASLt
//   stores depends on the call: a 16-bit C with its BIAS / GELU_BIAS
//   epilogue written directly; a 16-bit product (bias and int8 row scale
//   applied by hipBLASLt, the scale as its alpha vector) that the per-head
//   norm or the residual add + RMSNorm reads (round_product); otherwise the
//   fp32 product.  Operands are bf16, or -- with fp16 activations and the
//   caller's fp16 copy of the weights (w16_f16; int8 codes widened exactly,
//   bf16 weights rounded, sf_weights_to_f16, once per weight change) -- fp16,
//   and then the 16-bit outputs are fp16.  int8 weights without a copy are
//   multiplied directly by gemm_w8_tile_kernel when the call fits it (K =
//   2048, N a multiple of 256, fp16 activations, an fp16 product with act
//   NONE / GELU: every block projection of an int8 model at batch 32),
//   otherwise widened to bf16 codes in the workspace on every call.
//   single-pass path (no workspace): one workgroup of 8 waves per 16 or 64
//   weight rows over all of K, reduced in LDS, epilogue in place.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <atomic>
#include <map>
#include <mutex>
#include <tuple>

#include "sf_device.h"
#include "sf_hip.h"

#define SF_CHECK_OK(expr)                  \
    do {                                   \
        const int _st = (expr);            \
        if (_st != SF_OK) return _st;      \
    } while (0)

namespace sfk {

constexpr int kGemmThreads = 512;   // 8 waves

// Activation (A operand) element kinds.  bf16: as loaded.  fp32: a bf16
// (hi, lo) pair, two MFMAs per weight fragment.  fp16: fp16 MFMAs, with the
// bf16 weight fragment converted to fp16 in registers (exact for bf16
// magnitudes in [2^-14, 65504], to within 2^-25 below; int8 codes exact).
// kActF16W16 (split-K path only): fp16 activations and the caller's fp16
// copy of the weights (2 bytes per weight, loaded as bf16 weights are),
// used as MFMA operands as they are -- the same operands kActF16 forms in
// registers from bf16 weights or int8 codes, so the same products.
enum ActKind { kActBF16 = 0, kActF32 = 1, kActF16 = 2, kActF16W16 = 3 };

struct GemmArgs {
    const void* a;         // [M][lda] bf16, fp32 or fp16 (ActKind)
    const void* w;         // [N][ldw] bf16 or int8
    const float* w_scale;  // [N] (int8 weights)
    const float* bias;     // [N] or null
    void* c;               // [M][ldc] bf16 / f32
    int64_t lda, ldw, ldc;
    int M, N, K;
    int act;               // 0 none, 1 GELU(tanh), 2 SiLU
    int c_f32;
    int c_f16;             // fp16 C (else bf16 when !c_f32)
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
    // GeluOp, src/backend/cuda/ops/elementwise.cuh:35-54: 0.5 x (1 + tanh u),
    // u = sqrt(2 / pi) (x + 0.044715 x^3), evaluated as x / (1 + e^(-2u))
    // (0.5 (1 + tanh u) = 1 / (1 + e^(-2u))): one hardware exp2 and one
    // reciprocal, ~1 ulp each; x -> -inf gives -0, x -> +inf gives x.
    const float kAlpha = 0.7978845608028654f;
    const float kBeta = 0.044715f;
    const float kM2Log2e = -2.f * 1.4426950408889634f;
    const float u = kAlpha * (x + kBeta * x * x * x);
    return x * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(kM2Log2e * u));
}

__device__ __forceinline__ float silu(float x) { return x / (1.f + expf(-x)); }

__device__ __forceinline__ float apply_act(int act, float v) {
    return act == 1 ? gelu_tanh(v) : (act == 2 ? silu(v) : v);
}

// Eight bf16 weights -> fp16x8 (round to nearest; exact in fp16's normal range).
__device__ __forceinline__ f16x8 bf16x8_to_f16x8(u32x4 w) {
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = pack_f16x2_rn(__uint_as_float(w[e] << 16), __uint_as_float(w[e] & 0xffff0000u));
    return u32x4_as_f16x8(o);
}

// Eight int8 codes -> fp16x8 (exact).  (Building 1024 + (code + 128) as an
// fp16 bit pattern with one byte permute per two codes and subtracting 1152
// in packed fp16 is exact too, but made the int8 batch-1 loop slower:
// 11.83 vs 11.75 ms.)
__device__ __forceinline__ f16x8 i8x8_to_f16x8(uint2 raw) {
    u32x4 o;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const uint32_t src = p < 2 ? raw.x : raw.y;
        const int sh = (p & 1) * 16;
        o[p] = pack_f16x2_rn((float)(int)(int8_t)(src >> sh), (float)(int)(int8_t)(src >> (sh + 8)));
    }
    return u32x4_as_f16x8(o);
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

// An fp32 activation x as a bf16 pair: hi = bf16(x) (nearest), lo =
// bf16(x - hi); hi + lo carries ~16 significant bits of x, and
// W.hi + W.lo on two bf16 MFMAs is the product with that activation.
__device__ __forceinline__ void split_bf16x4(u32x4 f, uint2& hi, uint2& lo) {
    const float x0 = __uint_as_float(f[0]), x1 = __uint_as_float(f[1]);
    const float x2 = __uint_as_float(f[2]), x3 = __uint_as_float(f[3]);
    hi.x = pack_bf16x2(x0, x1);
    hi.y = pack_bf16x2(x2, x3);
    lo.x = pack_bf16x2(x0 - bf16_bits_to_f32(hi.x & 0xffffu), x1 - bf16_bits_to_f32(hi.x >> 16));
    lo.y = pack_bf16x2(x2 - bf16_bits_to_f32(hi.y & 0xffffu), x3 - bf16_bits_to_f32(hi.y >> 16));
}

// NR weight rows per workgroup: 16 (plain epilogue, K split 8 ways) or 64
// (one attention head, K split 2 ways, per-head epilogue).  MB activation
// blocks of 16 rows.  W8: int8 weights.  AK: activation kind (ActKind).
template <int NR, int MB, bool W8, int AK>
__global__ __launch_bounds__(kGemmThreads) void gemm_smallm_kernel(const GemmArgs g) {
    constexpr bool A32 = AK == kActF32;
    constexpr bool A16 = AK == kActF16;
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
    constexpr int AB = A32 ? 4 : 2;
    const __amdgpu_buffer_rsrc_t ars = make_rsrc(static_cast<const char*>(g.a) + (int64_t)m0 * g.lda * AB,
                                                 (uint32_t)((int64_t)max(0, min(MR, g.M - m0)) * g.lda * AB));
    // Rows past N (and activation rows past M) read as zeros.
    const uint32_t wrow_off = wrow < g.N ? (uint32_t)((int64_t)wrow * g.ldw * wbytes) : 0x80000000u;

    f32x4 acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};

    constexpr int U = A32 ? 4 : 8;   // chunks in flight per wave
    for (int c0 = c_beg; c0 < c_end; c0 += U) {
        bf16x8 wv[U];
        f16x8 wh[A16 ? U : 1];
        bf16x8 av[U][MB];
        bf16x8 al[A32 ? U : 1][MB];
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const int c = c0 + j;
            const bool live = c < c_end;
            const int k = 32 * c + 8 * g4;
            if constexpr (W8) {
                const uint32_t off = live ? wrow_off + (uint32_t)k : 0x80000000u;
                const uint2 raw = __builtin_bit_cast(
                    uint2, __builtin_amdgcn_raw_buffer_load_b64(wrs, off, 0, 0));
                if constexpr (A16) wh[j] = i8x8_to_f16x8(raw);
                else wv[j] = i8x8_to_bf16x8(raw);
            } else {
                const uint32_t off = live ? wrow_off + (uint32_t)k * 2 : 0x80000000u;
                const u32x4 raw = buffer_load16(wrs, off);
                if constexpr (A16) wh[j] = bf16x8_to_f16x8(raw);
                else wv[j] = __builtin_bit_cast(bf16x8, raw);
            }
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const uint32_t off = live ? (uint32_t)(((16 * mb + r) * g.lda + k) * AB) : 0x80000000u;
                if constexpr (A32) {
                    uint2 h0, l0, h1, l1;
                    split_bf16x4(buffer_load16(ars, off), h0, l0);
                    split_bf16x4(buffer_load16(ars, live ? off + 16 : 0x80000000u), h1, l1);
                    av[j][mb] = u32x4_as_bf16x8(u32x4{h0.x, h0.y, h1.x, h1.y});
                    al[j][mb] = u32x4_as_bf16x8(u32x4{l0.x, l0.y, l1.x, l1.y});
                } else {
                    av[j][mb] = __builtin_bit_cast(bf16x8, buffer_load16(ars, off));
                }
            }
        }
#pragma unroll
        for (int j = 0; j < U; ++j) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                if constexpr (A16) {
                    acc[mb] = mfma16x16x32_f16(wh[j], __builtin_bit_cast(f16x8, av[j][mb]), acc[mb]);
                } else {
                    acc[mb] = mfma16x16x32(wv[j], av[j][mb], acc[mb]);
                    if constexpr (A32) acc[mb] = mfma16x16x32(wv[j], al[j][mb], acc[mb]);
                }
            }
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
            } else if (g.c_f16) {
                reinterpret_cast<_Float16*>(g.c)[off] = (_Float16)v;
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

// ---------------------------------------------------------------------------
// split-K path
// ---------------------------------------------------------------------------
constexpr int kSkMaxSplits = 16;

struct SkArgs {
    const void* a;         // [M][lda] bf16, fp32 or fp16 (ActKind)
    const void* w;         // [N][ldw] bf16 or int8
    float* part;           // [splits][M][N] fp32
    int64_t lda, ldw;
    int M, N, K;
};

// LDS barrier that leaves outstanding global loads in flight (a plain
// __syncthreads also waits for every vector-memory load of the wave).

// Sum over the 64 lanes of a wave: the row sums, then the rows paired by
// v_permlane16_swap and v_permlane32_swap (VALU lane swaps of gfx950).
__device__ __forceinline__ float wave_sum(float x) {
    x = row16_sum(x);
    auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(s[0]) + __uint_as_float(s[1]);
    s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Workgroup (blockIdx.x, blockIdx.y, blockIdx.z) = (16*NW*NB-row weight
// tile, KT-wide K slice, 16*MB-row activation tile); NW waves share the LDS
// copy of the activation slice, and each wave contracts NB 16-row weight
// blocks against every activation fragment it reads from LDS.  Lane
// (g4 = lane/16, r = lane%16) of wave w supplies weight rows
// 16(NB w + nb) + r and activation row 16mb + r, k = 32t + 8g4 .. +7 of MFMA
// step t; accumulator [nb][mb] holds C^T[16(NB w + nb) + 4g4 + i][16mb + r].
// AK (ActKind): fp32 activations are staged in LDS as two bf16 planes (hi,
// lo) and contracted with two MFMAs per weight fragment; fp16 activations
// run fp16 MFMAs on weight fragments converted in registers.
template <int MB, int KT, int NW, bool W8, int NB, int AK>
__global__ __launch_bounds__(64 * NW) void gemm_splitk_kernel(const SkArgs g) {
    static_assert(!(W8 && AK == kActF16W16), "an fp16 weight copy is 2 bytes per weight");
    constexpr bool A32 = AK == kActF32;
    constexpr bool A16 = AK == kActF16 || AK == kActF16W16;
    constexpr bool WH = AK == kActF16W16;
    constexpr int kSkThreads = 64 * NW;
    constexpr int kSkRows = 16 * NW * NB;     // weight rows (output columns) per workgroup
    constexpr int MR = 16 * MB;
    constexpr int PITCH = 2 * KT + 16;       // bytes per LDS activation row (+16: bank shift)
    constexpr int AB = A32 ? 4 : 2;          // bytes per activation element in memory
    constexpr int CH = KT * AB / 16;         // 16-byte chunks per activation row
    constexpr int NCH = MR * CH;
    constexpr int PER = (NCH + kSkThreads - 1) / kSkThreads;
    constexpr int STEPS = KT / 32;
    constexpr int PLANES = A32 ? 2 : 1;
    __shared__ __attribute__((aligned(16))) char lds[PLANES * MR * PITCH];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int g4 = lane >> 4;
    const int r = lane & 15;
    const int nw = blockIdx.x * kSkRows;
    const int k0 = blockIdx.y * KT;
    const int m0 = blockIdx.z * MR;
    const int nsteps = min(KT, g.K - k0) / 32;

    // activation slice first (needed first); rows past M read as zeros
    const int mrows = min(MR, g.M - m0);
    const __amdgpu_buffer_rsrc_t ars =
        make_rsrc(static_cast<const char*>(g.a) + (int64_t)m0 * g.lda * AB, (uint32_t)((int64_t)mrows * g.lda * AB));
    u32x4 av[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int c = tid + kSkThreads * i;
        const int row = c / CH;
        const int k = k0 + (16 / AB) * (c % CH);
        const uint32_t off = (c < NCH && k < g.K) ? (uint32_t)((row * g.lda + k) * AB) : 0x80000000u;
        av[i] = buffer_load16(ars, off);
    }
    // every weight fragment of this wave in flight at once (non-temporal
    // cache policy: each weight byte is read once per step); rows past N read 0
    constexpr int WB = W8 ? 1 : 2;
    const int wrows = min(kSkRows, g.N - nw);
    const __amdgpu_buffer_rsrc_t wrs =
        make_rsrc(static_cast<const char*>(g.w) + (int64_t)nw * g.ldw * WB,
                  (uint32_t)((int64_t)wrows * g.ldw * WB));
    // wave w owns weight rows 16 (NB w + nb) + r, nb < NB: each activation
    // fragment read from LDS feeds NB MFMAs
    u32x4 wv[NB][W8 ? 1 : STEPS];
    uint2 wq[NB][W8 ? STEPS : 1];
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
        const int k = k0 + 32 * t + 8 * g4;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const uint32_t wrow_off = (uint32_t)((16 * (NB * w + nb) + r) * g.ldw * WB);
            const uint32_t off = t < nsteps ? wrow_off + (uint32_t)(k * WB) : 0x80000000u;
            if constexpr (W8)
                wq[nb][t] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(wrs, off, 0, 2));
            else
                wv[nb][t] = __builtin_amdgcn_raw_buffer_load_b128(wrs, off, 0, 2);
        }
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int c = tid + kSkThreads * i;
        if (c < NCH) {
            if constexpr (A32) {
                uint2 hi, lo;
                split_bf16x4(av[i], hi, lo);
                char* dst = lds + (c / CH) * PITCH + (c % CH) * 8;
                *reinterpret_cast<uint2*>(dst) = hi;
                *reinterpret_cast<uint2*>(dst + MR * PITCH) = lo;
            } else {
                *reinterpret_cast<u32x4*>(lds + (c / CH) * PITCH + (c % CH) * 16) = av[i];
            }
        }
    }
    lds_barrier();

    f32x4 acc[NB][MB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
        if (t < nsteps) {
            bf16x8 wf[NB];
            f16x8 wh[A16 ? NB : 1];
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                if constexpr (WH) {
                    wh[nb] = u32x4_as_f16x8(wv[nb][t]);
                } else if constexpr (A16) {
                    if constexpr (W8) wh[nb] = i8x8_to_f16x8(wq[nb][t]);
                    else wh[nb] = bf16x8_to_f16x8(wv[nb][t]);
                } else {
                    if constexpr (W8) wf[nb] = i8x8_to_bf16x8(wq[nb][t]);
                    else wf[nb] = __builtin_bit_cast(bf16x8, wv[nb][t]);
                }
            }
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const char* ap = lds + (16 * mb + r) * PITCH + (32 * t + 8 * g4) * 2;
                if constexpr (A16) {
                    const f16x8 ah = *reinterpret_cast<const f16x8*>(ap);
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb) acc[nb][mb] = mfma16x16x32_f16(wh[nb], ah, acc[nb][mb]);
                    continue;
                }
                const bf16x8 af = *reinterpret_cast<const bf16x8*>(ap);
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) acc[nb][mb] = mfma16x16x32(wf[nb], af, acc[nb][mb]);
                if constexpr (A32) {
                    const bf16x8 al = *reinterpret_cast<const bf16x8*>(ap + MR * PITCH);
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb) acc[nb][mb] = mfma16x16x32(wf[nb], al, acc[nb][mb]);
                }
            }
        }
    }

    float* P = g.part + (int64_t)blockIdx.y * g.M * g.N;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const int n = nw + 16 * (NB * w + nb) + 4 * g4;
        if (n < g.N) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const int m = m0 + 16 * mb + r;
                if (m < g.M) *reinterpret_cast<f32x4*>(P + (int64_t)m * g.N + n) = acc[nb][mb];
            }
        }
    }
}

struct EpiArgs {
    const float* part;     // [splits][M][N]
    const uint16_t* part16;  // or the library path's 16-bit product [M][ld16], bias and scale already in
    int64_t ld16;            // row stride of part16 (elements)
    int part16_f16;          // part16 holds fp16 (else bf16)
    int heads16;             // heads outputs take 16-byte stores (8-aligned head_out, strides)
    int splits;
    int M, N;
    int64_t m_off;         // row of the outputs that partial row 0 belongs to
    const float* w_scale;  // [N] or null
    const float* bias;     // [N] or null
    int act;
    // plain
    void* c;
    int64_t ldc;
    int c_f32, c_f16, accumulate;
    // per-head
    int H, S;
    float eps;
    const float* head_gamma[3];
    uint16_t* head_out[3];
    int64_t head_sb[3], head_sh[3], head_ss[3];
    // residual add + RMSNorm
    const float* norm_gamma;
    void* norm_out;
    int64_t norm_ldo;
    int norm_f32, norm_f16;
    // deferred RMSNorm, producer side (SF_EPI_ADD_NORM with norm_ss): x * gamma
    // to norm_out and, per 64-column tile t, norm_ss[t][m] = sum of x^2
    float* norm_ss;
    // consumer side: the activation rows hold x * gamma of a deferred norm;
    // each output row m is scaled by rsqrt(sum_t row_ss[t][m] * row_inv_n +
    // row_eps) after the weight scale and before the bias
    const float* row_ss;
    int row_tiles;
    float row_inv_n, row_eps;
};

// Sum of the K-slice partials for C[m][n..n+3], slices in ascending order,
// then scale, bias and activation.  Every load (all NS slices -- indices past
// `splits` re-read the last slice and are masked -- plus the bias and scale
// quads) is issued before the first add, so the epilogue costs one memory
// round trip.
// A 16-bit element (bf16, or fp16 when f16) as fp32.
__device__ __forceinline__ float bits16_to_f32(uint32_t h, int f16) {
    return f16 ? (float)__builtin_bit_cast(_Float16, (uint16_t)h) : bf16_bits_to_f32(h);
}

template <int NS>
struct Quad {
    f32x4 part[NS];
    f32x4 bias, scale;
};

template <int NS>
__device__ __forceinline__ void load_quad(const EpiArgs& e, int m, int n, Quad<NS>& q) {
    if (e.part16) {   // one "slice": the rounded product, bias and scale applied
        const uint2 h = *reinterpret_cast<const uint2*>(e.part16 + (int64_t)m * e.ld16 + n);
        q.part[0] = f32x4{bits16_to_f32(h.x & 0xffffu, e.part16_f16), bits16_to_f32(h.x >> 16, e.part16_f16),
                          bits16_to_f32(h.y & 0xffffu, e.part16_f16), bits16_to_f32(h.y >> 16, e.part16_f16)};
#pragma unroll
        for (int s = 1; s < NS; ++s) q.part[s] = q.part[0];
        q.bias = f32x4{0.f, 0.f, 0.f, 0.f};
        q.scale = f32x4{1.f, 1.f, 1.f, 1.f};
        return;
    }
    const float* p = e.part + (int64_t)m * e.N + n;
    const int64_t stride = (int64_t)e.M * e.N;
#pragma unroll
    for (int s = 0; s < NS; ++s)   // each partial is read once: non-temporal loads
        q.part[s] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p + min(s, e.splits - 1) * stride));
    q.bias = e.bias ? *reinterpret_cast<const f32x4*>(e.bias + n) : f32x4{0.f, 0.f, 0.f, 0.f};
    q.scale = e.w_scale ? *reinterpret_cast<const f32x4*>(e.w_scale + n) : f32x4{1.f, 1.f, 1.f, 1.f};
}

// rs: the row's deferred-norm scale (row_ss set), else unused.
template <int NS>
__device__ __forceinline__ f32x4 finish_quad(const EpiArgs& e, const Quad<NS>& q, float rs = 1.f) {
    f32x4 v = q.part[0];
#pragma unroll
    for (int s = 1; s < NS; ++s)
        if (s < e.splits) v += q.part[s];
    if (e.row_ss) {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = apply_act(e.act, deferred_affine(v[j], q.scale[j], rs, q.bias[j]));
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = apply_act(e.act, v[j] * q.scale[j] + q.bias[j]);
    }
    return v;
}

// The deferred-norm scale of row m for the 16 lanes that share it (lanes
// 16k .. 16k + 15, the reduce tiles' layout): lane j adds tiles j, j + 16,
// ... in ascending order, then the 16 lanes' sums are combined in a fixed
// butterfly (deterministic).  1 without row_ss.
__device__ __forceinline__ float deferred_row_scale(const EpiArgs& e, int m) {
    if (!e.row_ss) return 1.f;
    float t = 0.f;
    for (int k = (int)(threadIdx.x & 15); k < e.row_tiles; k += 16) t += e.row_ss[(int64_t)k * e.M + m];
    return deferred_rsqrt(row16_sum(t), e.row_inv_n, e.row_eps);
}

template <int NS>
__device__ __forceinline__ f32x4 finish4(const EpiArgs& e, int m, int n) {
    Quad<NS> q;
    load_quad<NS>(e, m, n, q);
    return finish_quad<NS>(e, q, deferred_row_scale(e, m));
}

__device__ __forceinline__ uint2 pack_bf16x4(f32x4 v) {
    return uint2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
}

__device__ __forceinline__ uint2 pack_16x4(f32x4 v, bool f16) {
    return f16 ? uint2{pack_f16x2_rn(v[0], v[1]), pack_f16x2_rn(v[2], v[3])} : pack_bf16x4(v);
}

// Output tile of a reduce workgroup when N % 64 == 0: 16 rows x the 64
// columns of one weight tile of the split-K kernel, tile index fastest.  That
// kernel writes every K slice of weight tile j from XCD j % 8 (workgroup id
// mod 8 is the XCD, and its grid's x extent N / 64 is a multiple of 8 for
// the model's N), so the reduce of tile j lands on the same XCD and reads
// those partials from its L2.  Lanes 16r .. 16r + 15 share row m.
__device__ __forceinline__ bool reduce_tile_rc(const EpiArgs& e, int& m, int& n) {
    const int ntl = e.N / 64;
    m = (int)(blockIdx.x / ntl) * 16 + (int)(threadIdx.x >> 4);
    n = 64 * (int)(blockIdx.x % ntl) + 4 * (int)(threadIdx.x & 15);
    return m < e.M;
}

template <int NS>
__global__ __launch_bounds__(256) void reduce_plain_kernel(const EpiArgs e) {
    int m, n;
    if ((e.N & 63) == 0) {
        if (!reduce_tile_rc(e, m, n)) return;
    } else {
        const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
        const int n4 = e.N / 4;
        if (idx >= (int64_t)e.M * n4) return;
        m = (int)(idx / n4);
        n = 4 * (int)(idx % n4);
    }
    f32x4 v = finish4<NS>(e, m, n);
    const int64_t off = (e.m_off + m) * e.ldc + n;
    if (e.c_f32) {
        f32x4* cp = reinterpret_cast<f32x4*>(static_cast<float*>(e.c) + off);
        if (e.accumulate) v += *cp;
        *cp = v;
    } else {
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(e.c) + off) = pack_16x4(v, e.c_f16);
    }
}

// 16 consecutive lanes hold the 64 columns of one head of one row.
template <int NS>
__global__ __launch_bounds__(256) void reduce_heads_kernel(const EpiArgs e) {
    int m, n;   // N % 64 == 0: a 16-lane group is one head of one row
    if (!reduce_tile_rc(e, m, n)) return;   // whole 16-lane groups
    f32x4 v = finish4<NS>(e, m, n);
    const int cols = e.H * 64;
    const int sec = n / cols;
    const int h = (n % cols) / 64;
    const int d = n % 64;
    const float* gamma = e.head_gamma[sec];
    if (gamma) {
        const f32x4 gq = *reinterpret_cast<const f32x4*>(gamma + d);
        // rms_norm_kernel_impl over the 64 head dims (norm.cuh:89-122)
        float ss = v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
        ss = row16_sum(ss);
        const float inv_rms = 1.f / sqrtf(ss / 64.f + e.eps);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = v[j] * inv_rms * gq[j];
    }
    const int64_t mg = e.m_off + m;
    const int64_t b = mg / e.S;
    const int64_t s = mg % e.S;
    uint16_t* o = e.head_out[sec] + b * e.head_sb[sec] + h * e.head_sh[sec] + s * e.head_ss[sec] + d;
    *reinterpret_cast<uint2*>(o) = pack_bf16x4(v);
}

// Per-head epilogue over the library path's bf16 product (bias and scale
// already in it): 8 lanes per (row, head), 8 columns each, so every lane
// moves 16 bytes each way; 256 threads = 32 rows x one 64-column head.
__global__ __launch_bounds__(256) void heads16_kernel(const EpiArgs e) {
    const int ntl = e.N / 64;
    const int m = (int)(blockIdx.x / ntl) * 32 + (int)(threadIdx.x >> 3);
    const int n = 64 * (int)(blockIdx.x % ntl) + 8 * (int)(threadIdx.x & 7);
    if (m >= e.M) return;   // whole 8-lane groups
    const u32x4 raw = *reinterpret_cast<const u32x4*>(e.part16 + (int64_t)m * e.ld16 + n);
    float v[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        v[2 * j] = bits16_to_f32(raw[j] & 0xffffu, e.part16_f16);
        v[2 * j + 1] = bits16_to_f32(raw[j] >> 16, e.part16_f16);
    }
    const int cols = e.H * 64;
    const int sec = n / cols;
    const int h = (n % cols) / 64;
    const int d = n % 64;
    const float* gamma = e.head_gamma[sec];
    if (gamma) {
        const f32x4 g0 = *reinterpret_cast<const f32x4*>(gamma + d);
        const f32x4 g1 = *reinterpret_cast<const f32x4*>(gamma + d + 4);
        // rms_norm_kernel_impl over the 64 head dims (norm.cuh:89-122)
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) ss += v[j] * v[j];
        ss += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(ss), 0xB1, 0xF, 0xF, true));   // quad_perm 1,0,3,2
        ss += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(ss), 0x4E, 0xF, 0xF, true));   // quad_perm 2,3,0,1
        ss += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(ss), 0x141, 0xF, 0xF, true));  // row_half_mirror
        const float inv_rms = 1.f / sqrtf(ss / 64.f + e.eps);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[j] = v[j] * inv_rms * g0[j];
            v[4 + j] = v[4 + j] * inv_rms * g1[j];
        }
    }
    const int64_t mg = e.m_off + m;
    const int64_t b = mg / e.S;
    const int64_t s = mg % e.S;
    uint16_t* o = e.head_out[sec] + b * e.head_sb[sec] + h * e.head_sh[sec] + s * e.head_ss[sec] + d;
    *reinterpret_cast<u32x4*>(o) =
        u32x4{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])};
}

// One workgroup of 512 threads per row: x[m] += result[m];
// out[m] = rmsnorm(x[m]) * gamma.
constexpr int kAddNormThreads = 512;
constexpr int kAddNormMaxChunks = 2;   // N <= 2 * 512 * 4 = 4096
template <int NS>
__global__ __launch_bounds__(kAddNormThreads) void reduce_addnorm_kernel(const EpiArgs e) {
    __shared__ float red[kAddNormThreads / 64];
    const int m = blockIdx.x;
    const int n4 = e.N / 4;
    float* x = static_cast<float*>(e.c) + (e.m_off + m) * e.ldc;
    // every load of the row first (partials and residual), then the stores:
    // a store to x between them would keep later loads from issuing early
    const int nch = min(kAddNormMaxChunks, (n4 - (int)threadIdx.x + kAddNormThreads - 1) / kAddNormThreads);
    Quad<NS> q[kAddNormMaxChunks];
    f32x4 xv[kAddNormMaxChunks], gv[kAddNormMaxChunks];
#pragma unroll
    for (int i = 0; i < kAddNormMaxChunks; ++i) {
        const int c = (int)threadIdx.x + kAddNormThreads * i;
        if (i < nch) {
            load_quad<NS>(e, m, 4 * c, q[i]);
            xv[i] = *reinterpret_cast<const f32x4*>(x + 4 * c);
            gv[i] = *reinterpret_cast<const f32x4*>(e.norm_gamma + 4 * c);
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < kAddNormMaxChunks; ++i) {
        if (i < nch) {
            xv[i] += finish_quad<NS>(e, q[i]);
            ss += xv[i][0] * xv[i][0] + xv[i][1] * xv[i][1] + xv[i][2] * xv[i][2] + xv[i][3] * xv[i][3];
        }
    }
#pragma unroll
    for (int i = 0; i < kAddNormMaxChunks; ++i)
        if (i < nch) *reinterpret_cast<f32x4*>(x + 4 * ((int)threadIdx.x + kAddNormThreads * i)) = xv[i];
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    lds_barrier();   // the residual stores above stay in flight
    float total = 0.f;
#pragma unroll
    for (int w = 0; w < kAddNormThreads / 64; ++w) total += red[w];
    const float inv_rms = 1.f / sqrtf(total / (float)e.N + e.eps);
#pragma unroll
    for (int i = 0; i < kAddNormMaxChunks; ++i) {
        const int c = threadIdx.x + kAddNormThreads * i;
        if (i < nch) {
            f32x4 o;
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = xv[i][j] * inv_rms * gv[i][j];
            const int64_t off = (e.m_off + m) * e.norm_ldo + 4 * c;
            if (e.norm_f32)
                *reinterpret_cast<f32x4*>(static_cast<float*>(e.norm_out) + off) = o;
            else
                *reinterpret_cast<uint2*>(static_cast<uint16_t*>(e.norm_out) + off) = pack_16x4(o, e.norm_f16);
        }
    }
}

// Deferred form of the residual add + RMSNorm, one workgroup per 16-row x
// 64-column tile (the reduce tiles' layout and XCD placement): x[m] +=
// result[m]; norm_out[m] = x[m] * gamma (not yet normalised); norm_ss[t][m]
// = the tile's sum of x^2 over its 64 columns (4 per lane in column order,
// then the 16 lanes of the row in a fixed butterfly).  The consumer of
// norm_out applies the row's rsqrt(mean x^2 + eps) after its contraction:
// (s a) W^T = s (a W^T).  Every CU takes part, where the row-wide form runs
// one workgroup per row.
template <int NS>
__global__ __launch_bounds__(256) void reduce_addnorm_cols_kernel(const EpiArgs e) {
    int m, n;
    if (!reduce_tile_rc(e, m, n)) return;   // whole 16-lane groups
    Quad<NS> q;
    load_quad<NS>(e, m, n, q);
    float* xp = static_cast<float*>(e.c) + (e.m_off + m) * e.ldc + n;
    f32x4 x = *reinterpret_cast<const f32x4*>(xp);
    const f32x4 gq = *reinterpret_cast<const f32x4*>(e.norm_gamma + n);
    x += finish_quad<NS>(e, q);
    *reinterpret_cast<f32x4*>(xp) = x;
    const f32x4 u = x * gq;
    const int64_t off = (e.m_off + m) * e.norm_ldo + n;
    if (e.norm_f32)
        *reinterpret_cast<f32x4*>(static_cast<float*>(e.norm_out) + off) = u;
    else
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(e.norm_out) + off) = pack_16x4(u, e.norm_f16);
    const float ss = row16_sum(x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3]);
    if ((threadIdx.x & 15) == 0) e.norm_ss[(int64_t)(n / 64) * e.M + m] = ss;
}

// int8 weight codes -> bf16 (exact), row-major [N][K] out of [N][ldw].
// CH codes per thread (16: one 16-byte load and two 16-byte stores, needs
// 16-byte aligned rows; 8 otherwise); 32-bit index arithmetic (callers keep
// N * K / CH below 2^31).
template <int CH>
__global__ __launch_bounds__(256) void widen_int8_kernel(const int8_t* __restrict__ q, int64_t ldw,
                                                         uint16_t* __restrict__ out, int N, int K) {
    const uint32_t idx = blockIdx.x * 256u + threadIdx.x;
    const uint32_t kc = (uint32_t)K / CH;
    if (idx >= (uint32_t)N * kc) return;
    const uint32_t n = idx / kc;
    const uint32_t k = CH * (idx - n * kc);
    const int8_t* src = q + (int64_t)n * ldw + k;
    uint16_t* dst = out + (int64_t)n * K + k;
    if constexpr (CH == 16) {
        const u32x4 raw = *reinterpret_cast<const u32x4*>(src);
        *reinterpret_cast<bf16x8*>(dst) = i8x8_to_bf16x8(uint2{raw[0], raw[1]});
        *reinterpret_cast<bf16x8*>(dst + 8) = i8x8_to_bf16x8(uint2{raw[2], raw[3]});
    } else {
        *reinterpret_cast<bf16x8*>(dst) = i8x8_to_bf16x8(*reinterpret_cast<const uint2*>(src));
    }
}

// Batched form: up to SF_CODES_MAX_JOBS matrices, 16 codes per thread;
// thread t belongs to the job whose [start[j], start[j+1]) holds t.
struct CodesJobs {
    const int8_t* q[SF_CODES_MAX_JOBS];
    uint16_t* out[SF_CODES_MAX_JOBS];
    int64_t ldq[SF_CODES_MAX_JOBS];
    int32_t K[SF_CODES_MAX_JOBS];
    uint32_t start[SF_CODES_MAX_JOBS + 1];
    int32_t count;
};

// Weight copies in fp16 for the library path's fp16 products: job j holds
// int8 codes (widened exactly) or bf16 weights (rounded to the nearest
// fp16: exact for 2^-14 <= |w| < 65520, to within 2^-25 below, +-inf
// beyond), 16 elements per thread; rows of K elements out of [N][ldq].
struct W16Jobs {
    const void* q[SF_CODES_MAX_JOBS];
    uint16_t* out[SF_CODES_MAX_JOBS];
    int64_t ldq[SF_CODES_MAX_JOBS];
    int32_t K[SF_CODES_MAX_JOBS];
    int32_t bf16[SF_CODES_MAX_JOBS];   // source bf16 (else int8)
    uint32_t start[SF_CODES_MAX_JOBS + 1];
    int32_t count;
};

__global__ __launch_bounds__(256) void weights_f16_kernel(const W16Jobs J) {
    const uint32_t idx = blockIdx.x * 256u + threadIdx.x;
    if (idx >= J.start[J.count]) return;
    int j = 0;
#pragma unroll
    for (int i = 1; i < SF_CODES_MAX_JOBS; ++i)
        if (i < J.count && idx >= J.start[i]) j = i;
    const uint32_t local = idx - J.start[j];
    const uint32_t kc = (uint32_t)J.K[j] / 16u;
    const uint32_t n = local / kc;
    const uint32_t k = 16u * (local - n * kc);
    uint16_t* dst = J.out[j] + (int64_t)n * J.K[j] + k;
    if (J.bf16[j]) {
        const u32x4* src = reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(J.q[j]) + (int64_t)n * J.ldq[j] + k);
        *reinterpret_cast<f16x8*>(dst) = bf16x8_to_f16x8(src[0]);
        *reinterpret_cast<f16x8*>(dst + 8) = bf16x8_to_f16x8(src[1]);
    } else {
        const u32x4 raw = *reinterpret_cast<const u32x4*>(static_cast<const int8_t*>(J.q[j]) + (int64_t)n * J.ldq[j] + k);
        *reinterpret_cast<f16x8*>(dst) = i8x8_to_f16x8(uint2{raw[0], raw[1]});
        *reinterpret_cast<f16x8*>(dst + 8) = i8x8_to_f16x8(uint2{raw[2], raw[3]});
    }
}

__global__ __launch_bounds__(256) void widen_jobs_kernel(const CodesJobs J) {
    const uint32_t idx = blockIdx.x * 256u + threadIdx.x;
    if (idx >= J.start[J.count]) return;
    int j = 0;
#pragma unroll
    for (int i = 1; i < SF_CODES_MAX_JOBS; ++i)
        if (i < J.count && idx >= J.start[i]) j = i;
    const uint32_t local = idx - J.start[j];
    const uint32_t kc = (uint32_t)J.K[j] / 16u;
    const uint32_t n = local / kc;
    const uint32_t k = 16u * (local - n * kc);
    const u32x4 raw = *reinterpret_cast<const u32x4*>(J.q[j] + (int64_t)n * J.ldq[j] + k);
    uint16_t* dst = J.out[j] + (int64_t)n * J.K[j] + k;
    *reinterpret_cast<bf16x8*>(dst) = i8x8_to_bf16x8(uint2{raw[0], raw[1]});
    *reinterpret_cast<bf16x8*>(dst + 8) = i8x8_to_bf16x8(uint2{raw[2], raw[3]});
}

struct SkPlan {
    bool split = false;
    int mb = 0, kt = 0, nw = 0, nb = 1, splits = 0, mtiles = 0, ntiles = 0;
    size_t ws_bytes = 0;
};

// Tile choice: one 64-row weight tile per workgroup and K slices of 256, so
// a 2048 x 2048 weight becomes 256 workgroups of 32 KB each and the
// 6144-row QKV weight 768 (three per CU: LDS <= 42 KB each, so the whole
// grid is resident at once).  The tile is two waves of two 16-row blocks:
// half the LDS fragment reads per output of four waves of one block
// (measured 0.7-1.2 us faster per call at M = 67-134; one wave of four
// blocks or two waves of four are slower).  Slices of 512 (four waves of
// one block) only when 256 would need more than 16 slices or more
// workgroups than fit on the chip at once for one 80-row tile.  The slicing depends on (N, K) only, never on M, so each
// row's sums are added in the same order whatever the batch: a row's result
// does not depend on how many rows share the call.  fp32 activations (a32)
// take two bf16 LDS planes: 84 KB for a 256-wide slice (one workgroup per
// CU), too much for a 512-wide one, so those shapes run single-pass.
constexpr int kSkResident = 256 * 3;
inline SkPlan plan_splitk(int M, int N, int K, bool a32) {
    SkPlan p;
    if (M <= 0 || M > 160 || N <= 0 || (N & 15) || K <= 0 || (K & 31)) return p;
    p.mb = M <= 80 ? (M + 15) / 16 : 5;
    p.mtiles = (M + 16 * p.mb - 1) / (16 * p.mb);
    p.nw = 2;
    p.nb = 2;
    p.ntiles = (N + 63) / 64;
    p.kt = 256;
    p.splits = (K + 255) / 256;
    if ((int64_t)p.ntiles * p.splits > kSkResident || p.splits > kSkMaxSplits) {
        p.kt = 512;
        p.nw = 4;
        p.nb = 1;
        p.splits = (K + 511) / 512;
    }
    if (p.splits > kSkMaxSplits) return SkPlan{};
    if (a32 && p.kt != 256) return SkPlan{};
    p.split = true;
    p.ws_bytes = (size_t)p.splits * M * N * 4;
    return p;
}

template <int KT, int NW, bool W8, int NB, int AK>
void launch_splitk_mb(const SkArgs& a, const SkPlan& p, hipStream_t s) {
    const dim3 grid(p.ntiles, p.splits, p.mtiles), block(64 * NW);
    switch (p.mb) {
        case 1: hipLaunchKernelGGL((gemm_splitk_kernel<1, KT, NW, W8, NB, AK>), grid, block, 0, s, a); break;
        case 2: hipLaunchKernelGGL((gemm_splitk_kernel<2, KT, NW, W8, NB, AK>), grid, block, 0, s, a); break;
        case 3: hipLaunchKernelGGL((gemm_splitk_kernel<3, KT, NW, W8, NB, AK>), grid, block, 0, s, a); break;
        case 4: hipLaunchKernelGGL((gemm_splitk_kernel<4, KT, NW, W8, NB, AK>), grid, block, 0, s, a); break;
        default: hipLaunchKernelGGL((gemm_splitk_kernel<5, KT, NW, W8, NB, AK>), grid, block, 0, s, a); break;
    }
}

template <bool W8>
void launch_splitk_w(const SkArgs& a, const SkPlan& p, int ak, hipStream_t s) {
    if (ak == kActF32) {
        launch_splitk_mb<256, 2, W8, 2, kActF32>(a, p, s);   // the plan keeps fp32 at 256-wide slices
    } else if (ak == kActF16) {
        if (p.kt == 256) launch_splitk_mb<256, 2, W8, 2, kActF16>(a, p, s);
        else launch_splitk_mb<512, 4, W8, 1, kActF16>(a, p, s);
    } else if (ak == kActF16W16) {
        if constexpr (!W8) {
            if (p.kt == 256) launch_splitk_mb<256, 2, false, 2, kActF16W16>(a, p, s);
            else launch_splitk_mb<512, 4, false, 1, kActF16W16>(a, p, s);
        }
    } else if (p.kt == 256) {
        launch_splitk_mb<256, 2, W8, 2, kActBF16>(a, p, s);
    } else {
        launch_splitk_mb<512, 4, W8, 1, kActBF16>(a, p, s);
    }
}

inline void launch_splitk(const SkArgs& a, const SkPlan& p, bool w8, int ak, hipStream_t s) {
    if (w8) launch_splitk_w<true>(a, p, ak, s);
    else launch_splitk_w<false>(a, p, ak, s);
}

template <int NS>
void launch_reduce(const sf_gemm_desc* d, const EpiArgs& e, hipStream_t s) {
    const int64_t quads = (int64_t)e.M * e.N / 4;
    const unsigned tiles = (unsigned)((int64_t)(e.N / 64) * ((e.M + 15) / 16));
    if (d->epilogue == SF_EPI_HEADS && e.part16 && e.heads16)
        hipLaunchKernelGGL(heads16_kernel, dim3((unsigned)((int64_t)(e.N / 64) * ((e.M + 31) / 32))), dim3(256), 0, s, e);
    else if (d->epilogue == SF_EPI_HEADS)
        hipLaunchKernelGGL(reduce_heads_kernel<NS>, dim3(tiles), dim3(256), 0, s, e);
    else if (d->epilogue == SF_EPI_ADD_NORM && e.norm_ss)
        hipLaunchKernelGGL(reduce_addnorm_cols_kernel<NS>, dim3(tiles), dim3(256), 0, s, e);
    else if (d->epilogue == SF_EPI_ADD_NORM)
        hipLaunchKernelGGL(reduce_addnorm_kernel<NS>, dim3(e.M), dim3(kAddNormThreads), 0, s, e);
    else if ((e.N & 63) == 0)
        hipLaunchKernelGGL(reduce_plain_kernel<NS>, dim3(tiles), dim3(256), 0, s, e);
    else
        hipLaunchKernelGGL(reduce_plain_kernel<NS>, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, s, e);
}

template <int NR, bool W8, int AK>
hipError_t launch_smallm(const GemmArgs& g, int mb, dim3 grid, hipStream_t s) {
    switch (mb) {
        case 1: hipLaunchKernelGGL((gemm_smallm_kernel<NR, 1, W8, AK>), grid, dim3(kGemmThreads), 0, s, g); break;
        case 2: hipLaunchKernelGGL((gemm_smallm_kernel<NR, 2, W8, AK>), grid, dim3(kGemmThreads), 0, s, g); break;
        case 3: hipLaunchKernelGGL((gemm_smallm_kernel<NR, 3, W8, AK>), grid, dim3(kGemmThreads), 0, s, g); break;
        case 4: hipLaunchKernelGGL((gemm_smallm_kernel<NR, 4, W8, AK>), grid, dim3(kGemmThreads), 0, s, g); break;
        default: hipLaunchKernelGGL((gemm_smallm_kernel<NR, 5, W8, AK>), grid, dim3(kGemmThreads), 0, s, g); break;
    }
    return hipGetLastError();
}

template <int NR, bool W8>
hipError_t launch_smallm_ak(const GemmArgs& g, int ak, int mb, dim3 grid, hipStream_t s) {
    if (ak == kActF32) return launch_smallm<NR, W8, kActF32>(g, mb, grid, s);
    if (ak == kActF16) return launch_smallm<NR, W8, kActF16>(g, mb, grid, s);
    return launch_smallm<NR, W8, kActBF16>(g, mb, grid, s);
}

template <int NR>
hipError_t launch_smallm_any(const GemmArgs& g, bool w8, int ak, int mb, dim3 grid, hipStream_t s) {
    return w8 ? launch_smallm_ak<NR, true>(g, ak, mb, grid, s) : launch_smallm_ak<NR, false>(g, ak, mb, grid, s);
}

// fp32 or fp16 activation rows -> bf16 (nearest) [rows][K] for the library path.
__global__ __launch_bounds__(256) void round_rows_bf16_kernel(const void* __restrict__ a, int a_f16, int64_t lda,
                                                               uint16_t* __restrict__ out, int rows, int K) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;   // 8 values per thread
    const int k8 = K / 8;
    if (idx >= (int64_t)rows * k8) return;
    const int64_t m = idx / k8;
    const int k = 8 * (int)(idx % k8);
    float x[8];
    if (a_f16) {
        const f16x8 h = *reinterpret_cast<const f16x8*>(static_cast<const _Float16*>(a) + m * lda + k);
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = (float)h[j];
    } else {
        const float* ap = static_cast<const float*>(a) + m * lda + k;
        const f32x4 x0 = *reinterpret_cast<const f32x4*>(ap);
        const f32x4 x1 = *reinterpret_cast<const f32x4*>(ap + 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            x[j] = x0[j];
            x[4 + j] = x1[j];
        }
    }
    *reinterpret_cast<u32x4*>(out + m * K + k) =
        u32x4{pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3]), pack_bf16x2(x[4], x[5]), pack_bf16x2(x[6], x[7])};
}

// ---------------------------------------------------------------------------
// int8 weights above 160 rows, read directly (no 16-bit copy of the weights)
// ---------------------------------------------------------------------------
// D[M][ldd] (fp16) = act(A[M][K] (fp16) . (q[N][K] * s[N])^T
// + bias[N]): dequantize_int8_fp16_kernel (quantization.cu:18-51) folded into
// the operand load -- every code widened exactly in registers, the row scale
// applied to the dot product -- with gemm_bias_act's BIAS / GELU_BIAS
// epilogue (cuda_backend.cu:337-467).
//
// One workgroup of 8 waves per 80-row x 256-column tile of D over the whole
// K, in kW8Chunks chunks of 128.  The activation chunk (80 x 128, 20 KB)
// goes HBM -> LDS by buffer_load ... lds (waves 0-3) into a 3-stage ring; a
// row's 16-byte pieces are XOR-swizzled by row % 16, so the fragment reads
// (16 rows x 16 B) hit distinct banks.  Wave w's 32 weight rows come straight
// into registers, two chunks ahead: lane (g4, r) loads codes k = 64 j +
// 16 g4 .. + 15 (j = 0, 1) of its two rows and widens them into the weight
// operands of MFMA steps (j, 0) and (j, 1); its activation fragment of step
// (j, h) is k = 64 j + 16 g4 + 8 h .. + 7, so every MFMA contracts the same
// 32 k of both operands (in an order a sum does not see).  Waits are explicit
// counts of the loads issued after the one waited for (chunks are issued in
// order and only those that exist), tied to the registers they fill; LDS
// reads are inline asm with their own lgkmcnt waits.
constexpr int kW8TileM = 80;
constexpr int kW8TileN = 256;
constexpr int kW8ChunkK = 128;
constexpr int kW8Chunks = 16;            // K = 2048 (the RDT-1B hidden size)
constexpr int kW8Stage = kW8TileM * kW8ChunkK * 2;   // 20 KB of activations
constexpr int kW8Ring = 3;
constexpr int kW8Lds = 82944;            // the ring plus slack: one workgroup per CU

template <int I>
struct IntC {
    static constexpr int value = I;
};

template <int C, int NCH, typename F>
__device__ __forceinline__ void for_chunks(F& f) {
    if constexpr (C < NCH) {
        f(IntC<C>{});
        for_chunks<C + 1, NCH>(f);
    }
}

__device__ __forceinline__ uint32_t lds_u32(const void* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const char*)(p);
}

// The five activation fragments of one MFMA step (rows 16 mb + r at
// addr + 4096 mb), no wait.
__device__ __forceinline__ void w8_read_a5(u32x4 (&o)[5], uint32_t addr) {
    asm volatile("ds_read_b128 %0, %5\n\t"
                 "ds_read_b128 %1, %5 offset:4096\n\t"
                 "ds_read_b128 %2, %5 offset:8192\n\t"
                 "ds_read_b128 %3, %5 offset:12288\n\t"
                 "ds_read_b128 %4, %5 offset:16384"
                 : "=&v"(o[0]), "=&v"(o[1]), "=&v"(o[2]), "=&v"(o[3]), "=&v"(o[4])
                 : "v"(addr)
                 : "memory");
}
template <int N>
__device__ __forceinline__ void w8_lgkm_wait5(u32x4 (&o)[5]) {
    asm volatile("s_waitcnt lgkmcnt(%5)" : "+v"(o[0]), "+v"(o[1]), "+v"(o[2]), "+v"(o[3]), "+v"(o[4]) : "n"(N) : "memory");
}
template <int N>
__device__ __forceinline__ void w8_vm_wait() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
template <int N>
__device__ __forceinline__ void w8_vm_wait4(u32x4 (&o)[4]) {
    asm volatile("s_waitcnt vmcnt(%4)" : "+v"(o[0]), "+v"(o[1]), "+v"(o[2]), "+v"(o[3]) : "n"(N) : "memory");
}
__device__ __forceinline__ void w8_barrier() { asm volatile("s_barrier" ::: "memory"); }
// 16 weight codes, a plain vector load whose wait is explicit.
__device__ __forceinline__ u32x4 w8_load16(u32x4 rsrc, uint32_t off) {
    u32x4 v;
    asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen" : "=v"(v) : "v"(off), "s"(rsrc) : "memory");
    return v;
}

// 16 int8 codes -> two fp16x8 (exact): 1024 + (code + 128) built as an fp16
// bit pattern by a byte permute, minus 1152 in packed fp16.
__device__ __forceinline__ void i8x16_to_f16(u32x4 raw, f16x8& h0, f16x8& h1) {
    uint32_t o[8];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const uint32_t x = raw[p] ^ 0x80808080u;
        f16x2v lo = __builtin_bit_cast(f16x2v, __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u));
        f16x2v hi = __builtin_bit_cast(f16x2v, __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u));
        lo = lo - f16x2v{(_Float16)1152.f, (_Float16)1152.f};
        hi = hi - f16x2v{(_Float16)1152.f, (_Float16)1152.f};
        o[2 * p] = __builtin_bit_cast(uint32_t, lo);
        o[2 * p + 1] = __builtin_bit_cast(uint32_t, hi);
    }
    h0 = u32x4_as_f16x8(u32x4{o[0], o[1], o[2], o[3]});
    h1 = u32x4_as_f16x8(u32x4{o[4], o[5], o[6], o[7]});
}

struct W8Args {
    const void* a;         // [M][lda] fp16, 16-byte aligned rows
    const int8_t* w;       // [N][ldw] codes, 16-byte aligned rows
    const float* scale;    // [N]
    const float* bias;     // [N] or null
    void* d;               // [M][ldd] fp16
    int64_t lda, ldw, ldd;
    int M, N, act;
    int mt, nt;            // tiles along M and N
    int xn, mper, nper;    // XCD blocks: 8 / xn row blocks of mper tiles x xn column blocks of nper
};

__global__ __launch_bounds__(512) void gemm_w8_tile_kernel(const W8Args g) {
    constexpr int MB = kW8TileM / 16, NB = 2, R = kW8Ring, NCH = kW8Chunks;
    constexpr int ADMA = kW8Stage / 1024 / 4;   // 5 DMA instructions per chunk in each of waves 0-3
    constexpr int WL = 2 * NB;                   // weight loads per lane and chunk
    constexpr int IT_D = ADMA + WL, IT_N = WL;   // loads per chunk: waves 0-3, waves 4-7
    __shared__ __attribute__((aligned(1024))) char ring[kW8Lds];
    static_assert(R * kW8Stage <= kW8Lds, "ring fits");

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g4 = lane >> 4, r = lane & 15;
    int tm, tn;
    if (g.xn == 0) {   // n fastest
        tm = (int)blockIdx.x / g.nt;
        tn = (int)blockIdx.x % g.nt;
    } else {
        // workgroup i runs on XCD i % 8: XCD x takes row block x / xn (mper
        // tiles) x column block x % xn (nper tiles), so each L2 fetches 1 / (8
        // / xn) of the activations and 1 / xn of the weights
        const int x = (int)blockIdx.x & 7, l = (int)blockIdx.x >> 3;
        if (l >= g.mper * g.nper) return;
        tm = (x / g.xn) * g.mper + l / g.nper;
        tn = (x % g.xn) * g.nper + l % g.nper;
    }
    if (tm >= g.mt || tn >= g.nt) return;
    const int m0 = tm * kW8TileM, n0 = tn * kW8TileN;
    const int mrows = min(kW8TileM, g.M - m0);
    const __amdgpu_buffer_rsrc_t ars =
        make_rsrc(static_cast<const char*>(g.a) + (int64_t)m0 * g.lda * 2, (uint32_t)((int64_t)mrows * g.lda * 2));
    // A DMA: instruction i of wave w < 4 fills stage bytes [1024 (ADMA w + i), + 1024):
    // row 4 (ADMA w + i) + lane / 16, its 16-byte piece (lane % 16) ^ (row % 16)
    uint32_t aoff[ADMA];
#pragma unroll
    for (int i = 0; i < ADMA; ++i) {
        const int row = 4 * (ADMA * (w & 3) + i) + (lane >> 4);
        aoff[i] = (uint32_t)((row * g.lda + 8 * ((lane & 15) ^ (row & 15))) * 2);
    }
    // weights: load 2 nb + j of lane (g4, r) reads row 32 w + 16 nb + r, codes 64 j + 16 g4 .. + 15
    uint32_t woff[WL];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int j = 0; j < 2; ++j)
            woff[2 * nb + j] = (uint32_t)((32 * w + 16 * nb + r) * g.ldw + 64 * j + 16 * g4);
    const uint64_t wbase = (uint64_t)(uintptr_t)g.w + (uint64_t)n0 * (uint64_t)g.ldw;
    const u32x4 wrs = {(uint32_t)wbase, (uint32_t)(wbase >> 32) & 0xffffu, (uint32_t)(kW8TileN * g.ldw),
                       0x00020000u};
    u32x4 wv[R][WL];
    auto issue = [&](int c, auto st_c) {
        constexpr int ST = decltype(st_c)::value;
        char* sa = ring + ST * kW8Stage;
        if (w < 4) {
#pragma unroll
            for (int i = 0; i < ADMA; ++i)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    ars, (__attribute__((address_space(3))) void*)(sa + (ADMA * w + i) * 1024), 16,
                    aoff[i] + (uint32_t)(c * kW8ChunkK * 2), 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < WL; ++i) wv[ST][i] = w8_load16(wrs, woff[i] + (uint32_t)(c * kW8ChunkK));
    };

    f32x4 acc[NB][MB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = f32x4{0.f, 0.f, 0.f, 0.f};

    const uint32_t lbase = lds_u32(ring);
    // activation fragment of step s = (j, h): row 16 mb + r, 16-byte piece 8 j + 2 g4 + h
    uint32_t aaddr[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int pc = 8 * (s >> 1) + 2 * g4 + (s & 1);
        aaddr[s] = lbase + r * (kW8ChunkK * 2) + ((pc ^ r) << 4);
    }
    issue(0, IntC<0>{});
    issue(1, IntC<1>{});

    auto mm = [&](const f16x8 (&wq)[NB], const u32x4 (&af)[5]) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) acc[nb][mb] = mfma16x16x32_f16(wq[nb], u32x4_as_f16x8(af[mb]), acc[nb][mb]);
    };

    auto body = [&](auto c_c) {
        constexpr int C = decltype(c_c)::value;
        constexpr int U = C % R;
        constexpr int LAST_BEFORE = (C + R - 2 < NCH - 1) ? C + R - 2 : NCH - 1;   // last chunk issued before this body
        constexpr int LAST_AFTER = (C + R - 1 < NCH - 1) ? C + R - 1 : NCH - 1;
        if (w < 4) w8_vm_wait<WL + IT_D * (LAST_BEFORE - C)>();   // this wave's DMA of chunk C
        w8_barrier();                                              // ... and every wave's, and stage (C - 1) % R read
        if constexpr (C + R - 1 < NCH) issue(C + R - 1, IntC<(U + R - 1) % R>{});
        const uint32_t so = U * kW8Stage;
        u32x4 a0[5], a1[5];
        w8_read_a5(a0, aaddr[0] + so);
        w8_read_a5(a1, aaddr[1] + so);
        if (w < 4) w8_vm_wait4<IT_D * (LAST_AFTER - C)>(wv[U]);   // the weight codes of chunk C
        else w8_vm_wait4<IT_N * (LAST_AFTER - C)>(wv[U]);
        f16x8 h0[NB], h1[NB];   // 16 codes -> the weight operands of steps (j, 0) and (j, 1)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) i8x16_to_f16(wv[U][2 * nb], h0[nb], h1[nb]);
        w8_lgkm_wait5<5>(a0);
        mm(h0, a0);
        w8_lgkm_wait5<0>(a1);
        w8_read_a5(a0, aaddr[2] + so);
        mm(h1, a1);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) i8x16_to_f16(wv[U][2 * nb + 1], h0[nb], h1[nb]);
        w8_read_a5(a1, aaddr[3] + so);
        w8_lgkm_wait5<5>(a0);
        mm(h0, a0);
        w8_lgkm_wait5<0>(a1);
        mm(h1, a1);
    };
    for_chunks<0, NCH>(body);
    w8_vm_wait<0>();

#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const int n = n0 + 16 * (NB * w + nb) + 4 * g4;
        const f32x4 sc = *reinterpret_cast<const f32x4*>(g.scale + n);
        const f32x4 bi = g.bias ? *reinterpret_cast<const f32x4*>(g.bias + n) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const int m = m0 + 16 * mb + r;
            if (m >= g.M) continue;
            f32x4 v;
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = apply_act(g.act, acc[nb][mb][i] * sc[i] + bi[i]);
            *reinterpret_cast<uint2*>(static_cast<uint16_t*>(g.d) + (int64_t)m * g.ldd + n) =
                uint2{pack_f16x2_rn(v[0], v[1]), pack_f16x2_rn(v[2], v[3])};
        }
    }
}

}  // namespace sfk

// ---------------------------------------------------------------------------
// library path (hipBLASLt)
// ---------------------------------------------------------------------------
namespace {

constexpr int kLibMinRows = 161;       // M above the split-K range
constexpr int kLibChunkRows = 8192;    // rows of fp32 product staged at once
constexpr size_t kLibLtBytes = 32u << 20;

size_t up256(size_t n) { return (n + 255) & ~(size_t)255; }

struct LibPlan {
    bool ok = false;
    int chunk = 0;
    size_t c_bytes = 0, w_bytes = 0, a_bytes = 0, total = 0;
};

// Workspace of the library path: the fp32 product of one chunk of rows, the
// bf16 copy of int8 weights, bf16 rows of an fp32 activation chunk, and
// hipBLASLt's own scratch.
LibPlan plan_library(int M, int N, int K, bool w8, bool a_conv) {
    LibPlan p;
    if (M < kLibMinRows || N <= 0 || (N & 15) || K <= 0 || (K & 31)) return p;
    p.chunk = std::min(M, kLibChunkRows);
    p.c_bytes = up256((size_t)p.chunk * N * 4);
    p.w_bytes = w8 ? up256((size_t)N * K * 2) : 0;
    p.a_bytes = a_conv ? up256((size_t)p.chunk * K * 2) : 0;
    p.total = p.c_bytes + p.w_bytes + p.a_bytes + kLibLtBytes;
    p.ok = true;
    return p;
}

// What hipBLASLt stores for one call: the fp32 product (all flags off), or
// a bf16 D with the bias epilogue (BIAS, or GELU_BIAS with gelu) and, for
// int8 weights, the per-row scale as a device alpha vector (one alpha per
// row of D, i.e. per output column n).  ldd: D's leading dimension.
// f16: fp16 operands (the activation and an fp16 weight copy) and, with
// out16, an fp16 D; otherwise bf16 operands and D.
struct LtKind {
    bool out16 = false, bias = false, gelu = false, alpha = false, f16 = false;
    int64_t ldd = 0;
    int bits() const {
        return (out16 ? 1 : 0) | (bias ? 2 : 0) | (gelu ? 4 : 0) | (alpha ? 8 : 0) | (f16 ? 16 : 0);
    }
};

// One hipBLASLt handle per device and one (descriptor, layouts, algorithm)
// per GEMM shape and kind, created on first use and kept for the process.
struct LtShape {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    LtKind kind;
    bool ok = false;
    int pick = -1;    // index of the algorithm in hipBLASLt's heuristic list (0: its first choice)
    int ncand = 0;    // usable candidates the heuristic returned
    bool timed = false;   // chosen by timing the candidates
};

std::mutex g_lt_mu;
std::map<int, hipblasLtHandle_t> g_lt_handles;
std::map<std::tuple<int, int, int, int, int64_t, int64_t, int64_t, int>, LtShape> g_lt_shapes;

// D = op(W) . A_act for one call; the bias pointer is a descriptor
// attribute, so setting it and enqueueing the product hold the lock (the
// descriptor is shared by every caller of the shape).
hipblasStatus_t lt_matmul(hipblasLtHandle_t h, const LtShape& sh, const hipblasLtMatmulAlgo_t& algo,
                          const float* bias, const float* alpha_vec, const void* W, const void* A, void* D,
                          void* ws, hipStream_t s) {
    std::lock_guard<std::mutex> lock(g_lt_mu);
    if (sh.kind.bias &&
        hipblasLtMatmulDescSetAttribute(sh.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof bias) !=
            HIPBLAS_STATUS_SUCCESS)
        return HIPBLAS_STATUS_INVALID_VALUE;
    const float one = 1.f, zero = 0.f;
    const void* alpha = sh.kind.alpha ? static_cast<const void*>(alpha_vec) : static_cast<const void*>(&one);
    return hipblasLtMatmul(h, sh.desc, alpha, W, sh.a, A, sh.b, &zero, D, sh.d, D, sh.d, &algo, ws, kLibLtBytes, s);
}

// Times each candidate algorithm on scratch buffers of the shape and
// returns the index of the fastest, or -1 when none ran.  A candidate runs
// back to back over nw distinct weight copies totalling more than the 256 MB
// memory-side cache (each read once, from HBM) with one activation and one
// output buffer, after two untimed calls: the state of a model step, which
// streams every layer's weights while the activations stay in cache.
// (Timing repeated calls on one warm weight, or single calls after a cache
// scrub, picked algorithms up to 35% slower in the denoise loop.)  Called
// from sf_gemm_prepare only, never under graph capture.
constexpr size_t kColdSetBytes = 320u << 20;

// Whether sf_gemm_prepare times the candidates (1, the default) or takes
// hipBLASLt's first heuristic candidate (0: the same algorithm in every
// process for a given library, GPU and shape; sf_gemm_set_algo_timing).
std::atomic<int> g_lt_timed{1};

int lt_pick_fastest(hipblasLtHandle_t h, const LtShape& sh, const hipblasLtMatmulHeuristicResult_t* res, int nres,
                    int N, int K, int rows, int64_t lda, int64_t ldw) {
    void *a = nullptr, *w = nullptr, *dbuf = nullptr, *ws = nullptr, *vec = nullptr;
    hipStream_t st = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int best = -1;
    float best_ms = 0.f;
    const size_t abytes = (size_t)rows * lda * 2, wbytes = (size_t)N * ldw * 2;
    const size_t dbytes = (size_t)rows * sh.kind.ldd * (sh.kind.out16 ? 2 : 4);
    size_t nw = std::min<size_t>(64, std::max<size_t>(2, (kColdSetBytes + wbytes - 1) / wbytes));
    bool ok = hipMalloc(&a, abytes) == hipSuccess && hipMalloc(&dbuf, dbytes) == hipSuccess &&
              hipMalloc(&ws, kLibLtBytes) == hipSuccess && hipMalloc(&vec, (size_t)N * 4) == hipSuccess &&
              hipStreamCreate(&st) == hipSuccess && hipEventCreate(&e0) == hipSuccess &&
              hipEventCreate(&e1) == hipSuccess;
    while (ok && nw > 2 && hipMalloc(&w, nw * wbytes) != hipSuccess) {   // fewer copies if memory is short
        (void)hipGetLastError();
        w = nullptr;
        nw /= 2;
    }
    ok = ok && (w || hipMalloc(&w, nw * wbytes) == hipSuccess);
    ok = ok && hipMemsetAsync(a, 0, abytes, st) == hipSuccess && hipMemsetAsync(w, 0, nw * wbytes, st) == hipSuccess &&
         hipMemsetAsync(vec, 0, (size_t)N * 4, st) == hipSuccess;
    if (ok) {
        const float* fv = static_cast<const float*>(vec);
        auto wi = [&](size_t i) { return static_cast<const void*>(static_cast<const char*>(w) + (i % nw) * wbytes); };
        for (int i = 0; i < nres; ++i) {
            if (res[i].state != HIPBLAS_STATUS_SUCCESS || res[i].workspaceSize > kLibLtBytes) continue;
            bool run = true;
            for (size_t r = 0; r < 2 && run; ++r)
                run = lt_matmul(h, sh, res[i].algo, fv, fv, wi(r), a, dbuf, ws, st) == HIPBLAS_STATUS_SUCCESS;
            run = run && hipEventRecord(e0, st) == hipSuccess;
            for (size_t r = 0; r < nw && run; ++r)
                run = lt_matmul(h, sh, res[i].algo, fv, fv, wi(r + 2), a, dbuf, ws, st) == HIPBLAS_STATUS_SUCCESS;
            run = run && hipEventRecord(e1, st) == hipSuccess && hipEventSynchronize(e1) == hipSuccess;
            float ms = 0.f;
            run = run && hipEventElapsedTime(&ms, e0, e1) == hipSuccess;
            if (run && (best < 0 || ms < best_ms)) {
                best = i;
                best_ms = ms;
            }
        }
    }
    if (st) (void)hipStreamSynchronize(st);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (st) (void)hipStreamDestroy(st);
    for (void* p : {a, w, dbuf, ws, vec})
        if (p) (void)hipFree(p);
    (void)hipGetLastError();
    return best;
}

// D ([rows][ldd], fp32 or bf16 per kind) = A_act (bf16 [rows][lda]) . W (bf16
// [N][ldw])^T (+ bias, GELU, alpha per kind), in hipBLASLt's column-major
// terms: D (N x rows, ld ldd) = op_T(W: K x N, ld ldw) . (A_act: K x rows,
// ld lda).  tune: choose among hipBLASLt's first 16 candidates by timing
// them (sf_gemm_prepare); otherwise its first choice.  A shape keeps the
// algorithm it was first created with.
int lt_lookup(int N, int K, int rows, int64_t lda, int64_t ldw, const LtKind& kind, hipblasLtHandle_t* h,
              const LtShape** out, bool tune = false) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return SF_EDEVICE;
    LtShape sh;
    {
        std::lock_guard<std::mutex> lock(g_lt_mu);
        auto hit = g_lt_handles.find(dev);
        if (hit == g_lt_handles.end()) {
            hipblasLtHandle_t nh = nullptr;
            if (hipblasLtCreate(&nh) != HIPBLAS_STATUS_SUCCESS) return SF_EDEVICE;
            hit = g_lt_handles.emplace(dev, nh).first;
        }
        *h = hit->second;
        auto it = g_lt_shapes.find(std::make_tuple(dev, N, K, rows, lda, ldw, kind.ldd, kind.bits()));
        if (it != g_lt_shapes.end()) {
            *out = &it->second;
            return it->second.ok ? SF_OK : SF_ENOTSUP;
        }
    }
    sh.kind = kind;
    bool ok = hipblasLtMatmulDescCreate(&sh.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS;
    const hipblasOperation_t opT = HIPBLAS_OP_T, opN = HIPBLAS_OP_N;
    ok = ok && hipblasLtMatmulDescSetAttribute(sh.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opT, sizeof opT) ==
                   HIPBLAS_STATUS_SUCCESS;
    ok = ok && hipblasLtMatmulDescSetAttribute(sh.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opN, sizeof opN) ==
                   HIPBLAS_STATUS_SUCCESS;
    if (kind.bias || kind.gelu) {
        const hipblasLtEpilogue_t epi = kind.bias ? (kind.gelu ? HIPBLASLT_EPILOGUE_GELU_BIAS : HIPBLASLT_EPILOGUE_BIAS)
                                                  : HIPBLASLT_EPILOGUE_GELU;
        ok = ok && hipblasLtMatmulDescSetAttribute(sh.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof epi) ==
                       HIPBLAS_STATUS_SUCCESS;
    }
    if (kind.bias) {
        const int32_t bt = HIP_R_32F;
        ok = ok && hipblasLtMatmulDescSetAttribute(sh.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof bt) ==
                       HIPBLAS_STATUS_SUCCESS;
    }
    if (kind.alpha) {
        const int32_t pm = HIPBLASLT_POINTER_MODE_ALPHA_DEVICE_VECTOR_BETA_HOST;
        ok = ok && hipblasLtMatmulDescSetAttribute(sh.desc, HIPBLASLT_MATMUL_DESC_POINTER_MODE, &pm, sizeof pm) ==
                       HIPBLAS_STATUS_SUCCESS;
    }
    const hipDataType t16 = kind.f16 ? HIP_R_16F : HIP_R_16BF;
    ok = ok && hipblasLtMatrixLayoutCreate(&sh.a, t16, K, N, ldw) == HIPBLAS_STATUS_SUCCESS;
    ok = ok && hipblasLtMatrixLayoutCreate(&sh.b, t16, K, rows, lda) == HIPBLAS_STATUS_SUCCESS;
    ok = ok && hipblasLtMatrixLayoutCreate(&sh.d, kind.out16 ? t16 : HIP_R_32F, N, rows, kind.ldd) ==
                   HIPBLAS_STATUS_SUCCESS;
    hipblasLtMatmulPreference_t pref = nullptr;
    ok = ok && hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS;
    const uint64_t wsmax = kLibLtBytes;
    ok = ok && hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsmax,
                                                     sizeof wsmax) == HIPBLAS_STATUS_SUCCESS;
    constexpr int kCand = 16;
    hipblasLtMatmulHeuristicResult_t res[kCand];
    int nres = 0;
    ok = ok && hipblasLtMatmulAlgoGetHeuristic(*h, sh.desc, sh.a, sh.b, sh.d, sh.d, pref, kCand, res, &nres) ==
                   HIPBLAS_STATUS_SUCCESS;
    // keep the candidates that ran the heuristic and fit the workspace
    int nuse = 0;
    for (int i = 0; ok && i < nres; ++i)
        if (res[i].state == HIPBLAS_STATUS_SUCCESS && res[i].workspaceSize <= kLibLtBytes) res[nuse++] = res[i];
    nres = nuse;
    ok = ok && nres > 0;
    if (pref) (void)hipblasLtMatmulPreferenceDestroy(pref);
    int pick = 0;   // hipBLASLt's first heuristic candidate unless timed
    if (ok && tune && g_lt_timed.load() && nres > 1) {
        const int best = lt_pick_fastest(*h, sh, res, nres, N, K, rows, lda, ldw);
        if (best >= 0) pick = best;
        sh.timed = true;
    }
    if (ok) {
        sh.algo = res[pick].algo;
        sh.pick = pick;
        sh.ncand = nres;
    }
    sh.ok = ok;
    std::lock_guard<std::mutex> lock(g_lt_mu);
    // a shape another thread created meanwhile wins; this one is dropped
    auto ins = g_lt_shapes.emplace(std::make_tuple(dev, N, K, rows, lda, ldw, kind.ldd, kind.bits()), sh);
    if (!ins.second) {
        if (sh.a) (void)hipblasLtMatrixLayoutDestroy(sh.a);
        if (sh.b) (void)hipblasLtMatrixLayoutDestroy(sh.b);
        if (sh.d) (void)hipblasLtMatrixLayoutDestroy(sh.d);
        if (sh.desc) (void)hipblasLtMatmulDescDestroy(sh.desc);
    }
    *out = &ins.first->second;
    return ins.first->second.ok ? SF_OK : SF_ENOTSUP;
}

}  // namespace

// ---------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------
namespace {
bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool al8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

int act_kind(const sf_gemm_desc* d) {
    return d->a_dtype == SF_F32 ? sfk::kActF32 : (d->a_dtype == SF_F16 ? sfk::kActF16 : sfk::kActBF16);
}

// The per-head outputs of an SF_EPI_HEADS descriptor (sections of H*64 of
// the N columns, at most 3; 8-byte aligned outputs and strides that are
// multiples of 4 elements, 16-byte / 8 for the 16-byte-store kernel).
int fill_heads(const sf_gemm_desc* d, sfk::EpiArgs& e) {
    if (d->H <= 0 || d->S <= 0) return SF_EINVAL;   // row m -> (m / S, m % S); a partial last element is fine
    const int cols = d->H * 64;
    if (d->N % cols || d->N / cols > 3) return SF_EINVAL;
    e.heads16 = 1;
    for (int j = 0; j < d->N / cols; ++j) {
        if (!d->head_out[j] || !al8(d->head_out[j])) return SF_EINVAL;
        if (!al16(d->head_out[j])) e.heads16 = 0;
        for (int q = 0; q < 3; ++q) {
            if (d->head_stride[j][q] & 3) return SF_EINVAL;
            if (d->head_stride[j][q] & 7) e.heads16 = 0;
        }
        e.head_out[j] = static_cast<uint16_t*>(d->head_out[j]);
        e.head_gamma[j] = d->head_gamma[j];
        e.head_sb[j] = d->head_stride[j][0];
        e.head_sh[j] = d->head_stride[j][1];
        e.head_ss[j] = d->head_stride[j][2];
    }
    e.H = d->H;
    e.S = d->S;
    return SF_OK;
}

// Shape / pointer checks shared by both paths; fills the epilogue fields.
int validate(const sf_gemm_desc* d, sfk::EpiArgs& e) {
    if (d->K == 0 || (d->K & 31)) return SF_ENOTSUP;
    if (d->a_dtype != SF_BF16 && d->a_dtype != SF_F32 && d->a_dtype != SF_F16) return SF_ENOTSUP;
    if (d->w_dtype != SF_BF16 && d->w_dtype != SF_I8) return SF_ENOTSUP;
    if (d->act < 0 || d->act > 2) return SF_EINVAL;
    if (!d->A || !d->W) return SF_EINVAL;
    if (!al16(d->A) || !al16(d->W) || (d->lda & 7) || d->lda < d->K) return SF_EINVAL;
    if ((d->ldw & 7) || d->ldw < d->K) return SF_EINVAL;
    if (d->w_dtype == SF_I8 && !d->w_scale) return SF_EINVAL;
    const int64_t abytes = d->a_dtype == SF_F32 ? 4 : 2;
    if ((int64_t)std::max(1, std::min(80, d->M)) * d->lda * abytes > 0x7fffffffLL) return SF_ENOTSUP;
    if ((int64_t)std::min(64, d->N) * d->ldw * 2 > 0x7fffffffLL) return SF_ENOTSUP;
    if (d->a_row_ss) {   // the activation rows hold x * gamma of a deferred norm
        if (d->epilogue != SF_EPI_PLAIN && d->epilogue != SF_EPI_HEADS) return SF_EINVAL;
        if (d->a_row_tiles < 1 || d->a_row_tiles > 64 || d->a_row_n <= 0 || !(d->a_row_eps >= 0.f)) return SF_EINVAL;
        if (d->N & 63) return SF_ENOTSUP;
        e.row_ss = d->a_row_ss;
        e.row_tiles = d->a_row_tiles;
        e.row_inv_n = 1.f / (float)d->a_row_n;
        e.row_eps = d->a_row_eps;
    }
    if (d->norm_ss) {    // deferred form of the residual add + RMSNorm
        if (d->epilogue != SF_EPI_ADD_NORM) return SF_EINVAL;
        if ((d->N & 63) || !al16(d->norm_ss)) return SF_ENOTSUP;
        e.norm_ss = d->norm_ss;
    }
    e.M = d->M;
    e.N = d->N;
    e.w_scale = d->w_dtype == SF_I8 ? d->w_scale : nullptr;
    e.bias = d->bias;
    e.act = d->act;
    e.eps = d->eps;
    if (d->epilogue == SF_EPI_HEADS) {
        SF_CHECK_OK(fill_heads(d, e));
    } else if (d->epilogue == SF_EPI_PARTIALS) {
        // no outputs besides the workspace
    } else if (d->epilogue == SF_EPI_PLAIN || d->epilogue == SF_EPI_ADD_NORM) {
        if (!d->C || d->ldc < d->N) return SF_EINVAL;
        if (d->c_dtype != SF_BF16 && d->c_dtype != SF_F32 && d->c_dtype != SF_F16) return SF_ENOTSUP;
        if ((d->accumulate || d->epilogue == SF_EPI_ADD_NORM) && d->c_dtype != SF_F32) return SF_EINVAL;
        e.c = d->C;
        e.ldc = d->ldc;
        e.c_f32 = d->c_dtype == SF_F32;
        e.c_f16 = d->c_dtype == SF_F16;
        e.accumulate = d->accumulate != 0 || d->epilogue == SF_EPI_ADD_NORM;
        if (d->epilogue == SF_EPI_ADD_NORM) {
            if (!d->norm_gamma || !d->norm_out || d->norm_ldo < d->N) return SF_EINVAL;
            if (d->norm_dtype != SF_BF16 && d->norm_dtype != SF_F32 && d->norm_dtype != SF_F16) return SF_ENOTSUP;
            if (d->N > 4096) return SF_ENOTSUP;
            e.norm_gamma = d->norm_gamma;
            e.norm_out = d->norm_out;
            e.norm_ldo = d->norm_ldo;
            e.norm_f32 = d->norm_dtype == SF_F32;
            e.norm_f16 = d->norm_dtype == SF_F16;
        }
    } else {
        return SF_EINVAL;
    }
    return SF_OK;
}

// The split path reads bias / scale / gamma and writes its outputs as
// 16-byte quads.
bool splittable(const sf_gemm_desc* d) {
    if (d->epilogue == SF_EPI_PARTIALS) return true;   // the kernel reads neither bias nor scale
    if (!al16(d->bias) || (d->w_dtype == SF_I8 && !al16(d->w_scale))) return false;
    if (d->epilogue == SF_EPI_HEADS) {
        for (int j = 0; j < 3; ++j)
            if (!al16(d->head_gamma[j])) return false;
        return true;
    }
    if (d->epilogue == SF_EPI_ADD_NORM && !al16(d->norm_gamma)) return false;
    if ((d->ldc & 3) || !(d->c_dtype == SF_F32 ? al16(d->C) : al8(d->C))) return false;
    if (d->epilogue == SF_EPI_ADD_NORM &&
        ((d->norm_ldo & 3) || !(d->norm_dtype == SF_F32 ? al16(d->norm_out) : al8(d->norm_out))))
        return false;
    return true;
}

int gemm_single_pass(const sf_gemm_desc* d, const sfk::EpiArgs& e, hipStream_t s) {
    // one buffer range covers the whole weight (32-bit byte offsets)
    const int64_t wbytes = d->w_dtype == SF_I8 ? 1 : 2;
    if ((int64_t)d->N * d->ldw * wbytes > 0x7fffffffLL) return SF_ENOTSUP;
    sfk::GemmArgs g{};
    g.a = d->A;
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
        for (int j = 0; j < 3; ++j) {
            g.head_out[j] = e.head_out[j];
            g.head_gamma[j] = e.head_gamma[j];
            g.head_sb[j] = e.head_sb[j];
            g.head_sh[j] = e.head_sh[j];
            g.head_ss[j] = e.head_ss[j];
        }
        g.heads = 1;
        g.H = e.H;
        g.S = e.S;
    } else {
        g.c = d->C;
        g.ldc = d->ldc;
        g.c_f32 = e.c_f32;
        g.c_f16 = e.c_f16;
        g.accumulate = e.accumulate;
    }
    const int mtiles = (d->M + 79) / 80;
    const int mb = d->M >= 80 ? 5 : (d->M + 15) / 16;
    const int ak = act_kind(d);
    hipError_t err;
    if (g.heads) {
        err = sfk::launch_smallm_any<64>(g, w8, ak, mb, dim3(d->N / 64, mtiles), s);
    } else {
        err = sfk::launch_smallm_any<16>(g, w8, ak, mb, dim3((d->N + 15) / 16, mtiles), s);
    }
    if (err != hipSuccess) return SF_ELAUNCH;
    if (d->epilogue == SF_EPI_ADD_NORM)
        return sf_rmsnorm(d->C, SF_F32, d->ldc, d->norm_gamma, d->norm_out, d->norm_dtype, d->norm_ldo,
                          d->M, d->N, d->eps, s);
    return SF_OK;
}
}  // namespace

// The split-K partial kernel over the descriptor's weights: W itself, or,
// with fp16 activations, the caller's fp16 copy when one is given
// (w16_f16 + w_codes16, [N][K]) -- the operands the kernel would otherwise
// form in registers, read without the conversion.
static int launch_splitk_desc(const sf_gemm_desc* d, sfk::SkArgs& a, const sfk::SkPlan& p, hipStream_t s) {
    if (d->a_dtype == SF_F16 && d->w16_f16 && d->w_codes16) {
        if (!al16(d->w_codes16)) return SF_EINVAL;
        a.w = d->w_codes16;
        a.ldw = d->K;
        sfk::launch_splitk(a, p, false, sfk::kActF16W16, s);
        return SF_OK;
    }
    a.w = d->W;
    a.ldw = d->ldw;
    sfk::launch_splitk(a, p, d->w_dtype == SF_I8, act_kind(d), s);
    return SF_OK;
}

// Leading dimensions hipBLASLt sees on the library path: int8 weights are
// widened into a [N][K] copy, fp32 activations rounded into [chunk][K].
// fp16 library path: fp16 activations with the caller's fp16 weight copy
// (w16_f16), multiplied by hipBLASLt in fp16 as they are.
bool lib_f16(const sf_gemm_desc* d) { return d->a_dtype == SF_F16 && d->w16_f16 != 0; }
int64_t lib_ldw(const sf_gemm_desc* d) { return (d->w_dtype == SF_I8 || lib_f16(d)) ? d->K : d->ldw; }
int64_t lib_lda(const sf_gemm_desc* d) { return (d->a_dtype != SF_BF16 && !lib_f16(d)) ? d->K : d->lda; }

// What the library path stores for this call.  A plain bf16 C (no
// accumulate, act NONE or GELU) is written by hipBLASLt itself with the bias
// (GELU_BIAS) epilogue -- one rounding, as on every path; with
// round_product the heads / add+norm epilogues read bf16(A.W^T + bias) from
// the workspace.  int8 row scales go in as hipBLASLt's alpha vector
// whenever D is bf16 (they must precede the rounding).  Otherwise the fp32
// product, and the epilogue kernel applies scale, bias and activation.
LtKind lib_kind(const sf_gemm_desc* d) {
    LtKind k;
    k.ldd = d->N;
    k.f16 = lib_f16(d);
    const bool act_ok = d->act == SF_ACT_NONE || d->act == SF_ACT_GELU_TANH;
    const bool plain16 = d->epilogue == SF_EPI_PLAIN && !d->accumulate && d->c_dtype == (k.f16 ? SF_F16 : SF_BF16);
    const bool rounded = (d->epilogue == SF_EPI_HEADS || d->epilogue == SF_EPI_ADD_NORM) && d->round_product;
    if (!act_ok || !(plain16 || rounded)) return k;
    k.out16 = true;
    k.bias = d->bias != nullptr;
    k.gelu = d->act == SF_ACT_GELU_TANH;
    k.alpha = d->w_dtype == SF_I8;
    if (plain16) k.ldd = d->ldc;
    return k;
}

// Whether hipBLASLt has an algorithm for every chunk shape of this call (a
// shape without one runs the single-pass kernel instead).
bool lib_available(const sf_gemm_desc* d, const LibPlan& lp, const LtKind& kind, bool tune) {
    hipblasLtHandle_t h;
    const LtShape* sh = nullptr;
    for (int rows : {lp.chunk, d->M % lp.chunk}) {
        if (rows <= 0) continue;
        if (lt_lookup(d->N, d->K, rows, lib_lda(d), lib_ldw(d), kind, &h, &sh, tune) != SF_OK) return false;
    }
    return true;
}

// A plain bf16 C that hipBLASLt writes itself needs no product buffer in
// the workspace.
bool lib_direct(const sf_gemm_desc* d) { return lib_kind(d).out16 && d->epilogue == SF_EPI_PLAIN; }
size_t lib_need(const sf_gemm_desc* d, const LibPlan& lp) { return lp.total - (lib_direct(d) ? lp.c_bytes : 0); }

// int8 weights above 160 rows without a 16-bit copy of the weights: the
// direct kernel (sfk::gemm_w8_tile_kernel) when the shape and the call fit
// it -- K = 2048, N a multiple of 256, fp16 activations, act NONE or GELU,
// and an fp16 product (a plain fp16 C, or round_product for the per-head /
// residual add + RMSNorm epilogues).
// Otherwise the library path widens the codes in the workspace per call.
bool w8_direct(const sf_gemm_desc* d) {
    if (d->w_dtype != SF_I8 || d->w_codes16) return false;
    if (d->a_dtype != SF_F16) return false;
    if (d->M < kLibMinRows || d->K != sfk::kW8Chunks * sfk::kW8ChunkK || d->N <= 0 || d->N % sfk::kW8TileN)
        return false;
    if ((d->ldw & 15) || (int64_t)sfk::kW8TileN * d->ldw > 0x7fffffffLL) return false;
    if (d->act != SF_ACT_NONE && d->act != SF_ACT_GELU_TANH) return false;
    const bool plain16 = d->epilogue == SF_EPI_PLAIN && !d->accumulate && d->c_dtype == d->a_dtype;
    const bool rounded = (d->epilogue == SF_EPI_HEADS || d->epilogue == SF_EPI_ADD_NORM) && d->round_product;
    return plain16 || rounded;
}

// The direct int8 product of rows [m0, m0 + rows) into D (ldd).
int launch_w8_direct(const sf_gemm_desc* d, int m0, int rows, void* D, int64_t ldd, hipStream_t s) {
    sfk::W8Args g{};
    g.a = static_cast<const char*>(d->A) + (int64_t)m0 * d->lda * 2;
    g.w = static_cast<const int8_t*>(d->W);
    g.scale = d->w_scale;
    g.bias = d->bias;
    g.d = D;
    g.lda = d->lda;
    g.ldw = d->ldw;
    g.ldd = ldd;
    g.M = rows;
    g.N = d->N;
    g.act = d->act;
    g.mt = (rows + sfk::kW8TileM - 1) / sfk::kW8TileM;
    g.nt = d->N / sfk::kW8TileN;
    // XCD blocks of 1/2 of the row tiles x 1/4 of the column tiles when the
    // columns divide (2144 x 2048 x 2048: 28.1 vs 28.6 us with n fastest)
    unsigned grid = (unsigned)(g.mt * g.nt);
    if (g.nt % 4 == 0) {
        g.xn = 4;
        g.nper = g.nt / g.xn;
        g.mper = (g.mt + 8 / g.xn - 1) / (8 / g.xn);
        grid = 8u * (unsigned)(g.mper * g.nper);
    }
    hipLaunchKernelGGL(sfk::gemm_w8_tile_kernel, dim3(grid), dim3(512), 0, s, g);
    return hipGetLastError() == hipSuccess ? SF_OK : SF_ELAUNCH;
}

extern "C" size_t sf_gemm_workspace_bytes(const sf_gemm_desc* d) {
    if (!d) return 0;
    const sfk::SkPlan p = sfk::plan_splitk(d->M, d->N, d->K, d->a_dtype == SF_F32);
    if (p.split) return p.ws_bytes;
    const LibPlan lp = plan_library(d->M, d->N, d->K, d->w_dtype == SF_I8, d->a_dtype != SF_BF16);
    return lp.ok ? lib_need(d, lp) : 0;
}

extern "C" int sf_gemm_prepare(const sf_gemm_desc* d) {
    if (!d) return SF_EINVAL;
    const LibPlan lp = plan_library(d->M, d->N, d->K, d->w_dtype == SF_I8, d->a_dtype != SF_BF16);
    if (!lp.ok) return SF_OK;   // split-K and single-pass paths need no setup
    // the fp32 product and the two bf16 products with bias (plain / GELU) at
    // D = [rows][N]; a shape hipBLASLt has no algorithm for is served by the
    // single-pass kernel: not an error
    LtKind k;
    k.ldd = d->N;
    k.f16 = lib_f16(d);
    (void)lib_available(d, lp, k, true);
    k.out16 = k.bias = true;
    k.alpha = d->w_dtype == SF_I8;
    (void)lib_available(d, lp, k, true);
    k.gelu = true;
    (void)lib_available(d, lp, k, true);
    return SF_OK;
}

extern "C" int sf_heads_bf16(const sf_gemm_desc* d, const void* P, int64_t ldp, void* stream) {
    if (!d || !P || d->epilogue != SF_EPI_HEADS || d->M < 0 || d->N <= 0 || (d->N & 63)) return SF_EINVAL;
    if (ldp < d->N || (ldp & 3) || !al8(P)) return SF_EINVAL;
    sfk::EpiArgs e{};
    SF_CHECK_OK(fill_heads(d, e));
    if (!d->M) return SF_OK;
    e.M = d->M;
    e.N = d->N;
    e.splits = 1;
    e.part16 = static_cast<const uint16_t*>(P);
    e.ld16 = ldp;
    e.act = SF_ACT_NONE;
    e.eps = d->eps;
    if (!al16(P) || (ldp & 7)) e.heads16 = 0;   // 16-byte rows for the 8-lane kernel
    hipStream_t s = static_cast<hipStream_t>(stream);
    sfk::launch_reduce<1>(d, e, s);
    return hipGetLastError() == hipSuccess ? SF_OK : SF_ELAUNCH;
}

extern "C" int sf_gemm_algo_pick(const sf_gemm_desc* d, int32_t* pick, int32_t* candidates, int32_t* timed) {
    if (!d || !pick) return SF_EINVAL;
    *pick = -1;
    if (candidates) *candidates = 0;
    if (timed) *timed = 0;
    const LibPlan lp = plan_library(d->M, d->N, d->K, d->w_dtype == SF_I8, d->a_dtype != SF_BF16 && !lib_f16(d));
    if (!lp.ok) return SF_ENOTSUP;   // not a library-path shape
    const LtKind kind = lib_kind(d);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return SF_EDEVICE;
    const int64_t ldw = (d->w_dtype == SF_I8 || lib_f16(d)) ? d->K : d->ldw;
    std::lock_guard<std::mutex> lock(g_lt_mu);
    auto it = g_lt_shapes.find(std::make_tuple(dev, d->N, d->K, lp.chunk, lib_lda(d), ldw, kind.ldd, kind.bits()));
    if (it == g_lt_shapes.end() || !it->second.ok) return SF_ENOTSUP;   // not prepared (or no algorithm)
    *pick = it->second.pick;
    if (candidates) *candidates = it->second.ncand;
    if (timed) *timed = it->second.timed ? 1 : 0;
    return SF_OK;
}

extern "C" int sf_gemm_set_algo_timing(int32_t timed) {
    if (timed != 0 && timed != 1) return SF_EINVAL;
    g_lt_timed.store(timed);
    return SF_OK;
}

extern "C" int32_t sf_gemm_int8_direct(const sf_gemm_desc* d) { return d && w8_direct(d) ? 1 : 0; }

extern "C" int32_t sf_gemm_num_splits(const sf_gemm_desc* d) {
    if (!d) return 0;
    const sfk::SkPlan p = sfk::plan_splitk(d->M, d->N, d->K, d->a_dtype == SF_F32);
    return p.split ? p.splits : 0;
}

extern "C" int sf_gemm(const sf_gemm_desc* d, void* stream) {
    if (!d) return SF_EINVAL;
    if (d->M < 0 || d->N < 0 || d->K < 0) return SF_EINVAL;
    if ((long)d->M * d->N == 0) return SF_OK;
    sfk::EpiArgs e{};
    SF_CHECK_OK(validate(d, e));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool a32 = d->a_dtype == SF_F32;
    const bool f16lib = lib_f16(d);   // library path in fp16 (the caller's fp16 weight copy)
    const bool a_conv = d->a_dtype != SF_BF16 && !f16lib;   // library path: activations rounded to bf16 first
    if (f16lib && (!d->w_codes16 || !al16(d->w_codes16))) return SF_EINVAL;
    if (a32 && ((d->lda & 3) || !al16(d->A))) return SF_EINVAL;
    const sfk::SkPlan p = sfk::plan_splitk(d->M, d->N, d->K, a32);
    // the deferred norm (either side) runs on the split-K path only
    if ((d->norm_ss || d->a_row_ss) && !(d->workspace && p.split && splittable(d))) return SF_ENOTSUP;
    if (d->epilogue == SF_EPI_PARTIALS) {   // the K-slice sums only, for a consumer to finish
        if (!p.split || !d->workspace) return SF_ENOTSUP;
        if (d->workspace_bytes < 0 || (size_t)d->workspace_bytes < p.ws_bytes) return SF_EWORKSPACE;
        if (!al16(d->workspace)) return SF_EINVAL;
        sfk::SkArgs a{};
        a.a = d->A;
        a.part = static_cast<float*>(d->workspace);
        a.lda = d->lda;
        a.M = d->M; a.N = d->N; a.K = d->K;
        SF_CHECK_OK(launch_splitk_desc(d, a, p, s));
        return hipGetLastError() == hipSuccess ? SF_OK : SF_ELAUNCH;
    }
    if (d->workspace && !p.split && splittable(d) && w8_direct(d)) {
        const LibPlan lp = plan_library(d->M, d->N, d->K, true, false);
        const bool plain = d->epilogue == SF_EPI_PLAIN;   // the kernel writes C
        const size_t need = plain ? 0 : (size_t)lp.chunk * d->N * 2;
        if (!lp.ok) return SF_ENOTSUP;
        if (d->workspace_bytes < 0 || (size_t)d->workspace_bytes < need) return SF_EWORKSPACE;
        if (!al16(d->workspace)) return SF_EINVAL;
        for (int m0 = 0; m0 < d->M; m0 += lp.chunk) {
            const int rows = std::min(lp.chunk, d->M - m0);
            if (plain) {
                SF_CHECK_OK(launch_w8_direct(d, m0, rows, static_cast<uint16_t*>(d->C) + (int64_t)m0 * d->ldc,
                                             d->ldc, s));
                continue;
            }
            SF_CHECK_OK(launch_w8_direct(d, m0, rows, d->workspace, d->N, s));
            sfk::EpiArgs ec = e;   // scale, bias and activation are in the 16-bit product
            ec.splits = 1;
            ec.M = rows;
            ec.m_off = m0;
            ec.part = nullptr;
            ec.part16 = static_cast<const uint16_t*>(d->workspace);
            ec.part16_f16 = 1;
            ec.ld16 = d->N;
            ec.bias = nullptr;
            ec.w_scale = nullptr;
            ec.act = SF_ACT_NONE;
            sfk::launch_reduce<1>(d, ec, s);
            if (hipGetLastError() != hipSuccess) return SF_ELAUNCH;
        }
        return SF_OK;
    }
    if (d->workspace && !p.split && splittable(d)) {
        const bool w8 = d->w_dtype == SF_I8;
        const LibPlan lp = plan_library(d->M, d->N, d->K, w8, a_conv);
        const LtKind kind = lib_kind(d);
        if (lp.ok && lib_available(d, lp, kind, false)) {
            const bool direct = kind.out16 && d->epilogue == SF_EPI_PLAIN;   // hipBLASLt writes C
            if (d->workspace_bytes < 0 || (size_t)d->workspace_bytes < lib_need(d, lp)) return SF_EWORKSPACE;
            if (!al16(d->workspace)) return SF_EINVAL;
            // [fp32 / bf16 product (not when direct)][int8 widened][activation rows][hipBLASLt]
            char* ws = static_cast<char*>(d->workspace);
            float* cbuf = reinterpret_cast<float*>(ws);
            const size_t c_bytes = direct ? 0 : lp.c_bytes;
            uint16_t* abuf = reinterpret_cast<uint16_t*>(ws + c_bytes + lp.w_bytes);
            void* ltws = ws + c_bytes + lp.w_bytes + lp.a_bytes;
            const void* W = d->W;
            int64_t ldw = d->ldw;
            if (f16lib) {   // the caller's fp16 copy (int8 codes or bf16 weights)
                W = d->w_codes16;
                ldw = d->K;
            } else if (w8 && d->w_codes16) {   // the caller's widened copy
                if (!al16(d->w_codes16)) return SF_EINVAL;
                W = d->w_codes16;
                ldw = d->K;
            } else if (w8) {
                uint16_t* wb = reinterpret_cast<uint16_t*>(ws + c_bytes);
                const bool c16 = (d->ldw & 15) == 0 && (d->K & 15) == 0;
                const int64_t nch = (int64_t)d->N * (d->K / (c16 ? 16 : 8));
                if (nch >= 0x7fffffffLL) return SF_ENOTSUP;
                const dim3 grid((unsigned)((nch + 255) / 256));
                if (c16)
                    hipLaunchKernelGGL(sfk::widen_int8_kernel<16>, grid, dim3(256), 0, s,
                                       static_cast<const int8_t*>(d->W), d->ldw, wb, d->N, d->K);
                else
                    hipLaunchKernelGGL(sfk::widen_int8_kernel<8>, grid, dim3(256), 0, s,
                                       static_cast<const int8_t*>(d->W), d->ldw, wb, d->N, d->K);
                if (hipGetLastError() != hipSuccess) return SF_ELAUNCH;
                W = wb;
                ldw = d->K;
            }
            for (int m0 = 0; m0 < d->M; m0 += lp.chunk) {
                const int rows = std::min(lp.chunk, d->M - m0);
                hipblasLtHandle_t h;
                const LtShape* sh = nullptr;
                SF_CHECK_OK(lt_lookup(d->N, d->K, rows, lib_lda(d), ldw, kind, &h, &sh));
                const uint16_t* Ac;
                if (a_conv) {
                    const int64_t n8 = (int64_t)rows * (d->K / 8);
                    const char* Ab = static_cast<const char*>(d->A) + (int64_t)m0 * d->lda * (a32 ? 4 : 2);
                    hipLaunchKernelGGL(sfk::round_rows_bf16_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256),
                                       0, s, static_cast<const void*>(Ab), a32 ? 0 : 1, d->lda, abuf, rows, d->K);
                    if (hipGetLastError() != hipSuccess) return SF_ELAUNCH;
                    Ac = abuf;
                } else {
                    Ac = static_cast<const uint16_t*>(d->A) + (int64_t)m0 * d->lda;
                }
                void* D = direct ? static_cast<void*>(static_cast<uint16_t*>(d->C) + (int64_t)m0 * d->ldc)
                                 : static_cast<void*>(cbuf);
                if (lt_matmul(h, *sh, sh->algo, d->bias, d->w_scale, W, Ac, D, ltws, s) != HIPBLAS_STATUS_SUCCESS)
                    return SF_ELAUNCH;
                if (direct) continue;
                sfk::EpiArgs ec = e;
                ec.splits = 1;
                ec.M = rows;
                ec.m_off = m0;
                if (kind.out16) {   // bias, GELU and the int8 scale are in the 16-bit product
                    ec.part = nullptr;
                    ec.part16_f16 = kind.f16 ? 1 : 0;
                    ec.part16 = reinterpret_cast<const uint16_t*>(cbuf);
                    ec.ld16 = d->N;
                    ec.bias = nullptr;
                    ec.w_scale = nullptr;
                    ec.act = SF_ACT_NONE;
                } else {
                    ec.part = cbuf;
                }
                sfk::launch_reduce<1>(d, ec, s);
                if (hipGetLastError() != hipSuccess) return SF_ELAUNCH;
            }
            return SF_OK;
        }
    }
    if (!d->workspace || !p.split || !splittable(d)) return gemm_single_pass(d, e, s);
    if (d->workspace_bytes < 0 || (size_t)d->workspace_bytes < p.ws_bytes) return SF_EWORKSPACE;
    if (!al16(d->workspace)) return SF_EINVAL;
    sfk::SkArgs a{};
    a.a = d->A;
    a.part = static_cast<float*>(d->workspace);
    a.lda = d->lda;
    a.M = d->M; a.N = d->N; a.K = d->K;
    SF_CHECK_OK(launch_splitk_desc(d, a, p, s));
    if (hipGetLastError() != hipSuccess) return SF_ELAUNCH;
    e.part = a.part;
    e.splits = p.splits;
    if (p.splits <= 1) sfk::launch_reduce<1>(d, e, s);
    else if (p.splits <= 4) sfk::launch_reduce<4>(d, e, s);
    else if (p.splits <= 8) sfk::launch_reduce<8>(d, e, s);
    else sfk::launch_reduce<16>(d, e, s);
    return hipGetLastError() == hipSuccess ? SF_OK : SF_ELAUNCH;
}

extern "C" int sf_weights_to_f16(const sf_w16_job* jobs, int32_t count, void* stream) {
    if (count == 0) return SF_OK;
    if (!jobs || count < 0 || count > SF_CODES_MAX_JOBS) return SF_EINVAL;
    sfk::W16Jobs J{};
    J.count = count;
    uint64_t total = 0;
    for (int j = 0; j < count; ++j) {
        const sf_w16_job& b = jobs[j];
        if (b.N < 0 || b.K < 0) return SF_EINVAL;
        if (b.w_dtype != SF_I8 && b.w_dtype != SF_BF16) return SF_EINVAL;
        J.start[j] = (uint32_t)total;
        if ((int64_t)b.N * b.K == 0) continue;
        const int64_t ldbytes = b.ldw * (b.w_dtype == SF_BF16 ? 2 : 1);
        if (!b.w || !b.out || !al16(b.w) || !al16(b.out) || (b.K & 15) || (ldbytes & 15) || b.ldw < b.K)
            return SF_EINVAL;
        J.q[j] = b.w;
        J.out[j] = static_cast<uint16_t*>(b.out);
        J.ldq[j] = b.ldw;
        J.K[j] = b.K;
        J.bf16[j] = b.w_dtype == SF_BF16;
        total += (uint64_t)b.N * (uint64_t)(b.K / 16);
        if (total >= 0x7fffff00ull) return SF_ENOTSUP;   // 32-bit thread indices
    }
    J.start[count] = (uint32_t)total;
    if (total == 0) return SF_OK;
    hipLaunchKernelGGL(sfk::weights_f16_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), J);
    return hipGetLastError() == hipSuccess ? SF_OK : SF_ELAUNCH;
}

extern "C" int sf_int8_codes_to_bf16(const sf_codes_job* jobs, int32_t count, void* stream) {
    if (count == 0) return SF_OK;
    if (!jobs || count < 0 || count > SF_CODES_MAX_JOBS) return SF_EINVAL;
    sfk::CodesJobs J{};
    J.count = count;
    uint64_t total = 0;
    for (int j = 0; j < count; ++j) {
        const sf_codes_job& b = jobs[j];
        if (b.N < 0 || b.K < 0) return SF_EINVAL;
        J.start[j] = (uint32_t)total;
        if ((int64_t)b.N * b.K == 0) continue;
        if (!b.q || !b.out || !al16(b.q) || !al16(b.out) || (b.K & 15) || (b.ldq & 15) || b.ldq < b.K)
            return SF_EINVAL;
        J.q[j] = b.q;
        J.out[j] = static_cast<uint16_t*>(b.out);
        J.ldq[j] = b.ldq;
        J.K[j] = b.K;
        total += (uint64_t)b.N * (uint64_t)(b.K / 16);
        if (total >= 0x7fffff00ull) return SF_ENOTSUP;   // 32-bit thread indices
    }
    J.start[count] = (uint32_t)total;
    if (total == 0) return SF_OK;
    hipLaunchKernelGGL(sfk::widen_jobs_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), J);
    return hipGetLastError() == hipSuccess ? SF_OK : SF_ELAUNCH;
}
