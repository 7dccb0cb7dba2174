// Attention for the RDT-1B denoise loop on MI355X (gfx950).
//
// Replaces the attention op behind IBackend::attention
// (include/servoflow/backend/backend.h:105-110): CUDABackend::attention
// (src/backend/cuda/cuda_backend.cu:470-501) -> cuda_ops::flash_attention
// (src/backend/cuda/ops/attention.cu:183-197), whose arithmetic is the
// online-softmax loop of naive_attention_kernel (attention.cu:90-139).
//
// Design (the ring kernel serves the 67 x 4374 / 67 x <=1024
// cross-attention; attn_short_kernel below serves key sets of <= 128, the
// 67 x 67 self-attention):
//   * grid = (splits x query-chunks, H, B); a workgroup of 4 waves owns one
//     (b, h, query chunk of 80 rows, key split); up to two fit on a CU.
//     Splitting the keys (flash-decoding) is what fills 256 CUs when
//     B*H = 32 and the keys are many (the image).  With at most 1024 keys
//     (the language) such grids run one 16-row query block per workgroup
//     over all keys instead (QB = 1: no split, no merge pass), a head's
//     blocks on one XCD so its K/V are fetched into that L2 once.
//   * K/V tiles of 128 keys are streamed HBM -> LDS by buffer_load ... lds
//     (16-byte, coalesced, no VGPR staging) into a two-stage ring, so the
//     next tile's loads are in flight while the current one is contracted;
//     V stays in its [key][d] layout and is read as V^T with
//     ds_read_b64_tr_b16.
//   * Each wave contracts 32 keys of the tile against all 80 query rows with
//     v_mfma_f32_16x16x32_bf16: S^T = K.Q^T, then O^T += V^T.P^T.  The S^T
//     accumulator layout (lane = query, 4 consecutive keys per lane) is
//     directly the B operand P^T, so no shuffle sits between the two
//     contractions.
//   * P.V runs in fp16 by default (V converted exactly in fp16's normal
//     range, to within 2^-25 below it, inf above 2^16; P rounded to the
//     nearest fp16); the exact form carries P as a
//     bf16 (hi, lo) pair against bf16 V (~16 mantissa bits of P: a single
//     bf16 P costs ~1.1e-3 mean relative error on its own, the whole 1e-3
//     budget).
//   * Online softmax in the log2 domain; the four waves' (m, l, O) merge in
//     LDS; multi-split partials merge in a second small kernel.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <mutex>

#include "sf_device.h"
#include "sf_hip.h"

namespace sfk {

constexpr int kD = 64;      // head dim this kernel family is built for
constexpr int kQB = 5;      // 16-row query blocks per workgroup (80 rows >= 67)
constexpr int kMaxSplits = 64;

struct AttnArgs {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    void* o;
    float* part_o;    // [B*H][nsplit][Sq][64] unnormalised outputs
    float* part_ml;   // [B*H][nsplit][Sq][2]  (running max in log2 units, sum)
    const int32_t* valid_len;
    const uint8_t* kv_mask;   // [B][kv_mask_stride] bytes, nonzero = attend
    int64_t kv_mask_stride;
    int64_t q_sb, q_sh, q_ss;
    int64_t k_sb, k_sh, k_ss;
    int64_t v_sb, v_sh, v_ss;
    int64_t o_sb, o_sh, o_ss;
    int B, H, Sq, Sk;
    int nsplit;
    int nqc;          // query chunks
    int out_kind;     // OutKind
    int causal;
    float scale_log2;   // scale * log2(e)
    // Q from split-K partials (the kQP instance): [q_splits][B*Sq][H*64]
    const float* qp;
    int q_splits;
    uint32_t qp_bytes;   // the partials' extent (buffer range)
    const float* q_bias;
    const float* q_scale;
    const float* q_gamma;   // per-head RMSNorm weight of Q (with or without partials)
    float q_eps;
    const float* k_gamma;   // per-head RMSNorm weight of K (the short-key kernel)
    int q_f16;              // bf16 instances: Q rows given in fp16, rounded to bf16 (after q_gamma) on load
    // Q from partials of x * gamma rows (a deferred RMSNorm): row scale from
    // q_row_ss[t][b * Sq + s], t < q_row_tiles
    const float* q_row_ss;
    int q_row_tiles;
    float q_row_inv_n, q_row_eps;
};

enum OutKind { kOutBF16 = 0, kOutF32 = 1, kOutF16 = 2 };

__device__ __forceinline__ void store_out(const AttnArgs& a, int b, int h, int q,
                                          int d, float val) {
    const int64_t off = b * a.o_sb + h * a.o_sh + q * a.o_ss + d;
    if (a.out_kind == kOutF32) {
        reinterpret_cast<float*>(a.o)[off] = val;
    } else if (a.out_kind == kOutF16) {
        reinterpret_cast<_Float16*>(a.o)[off] = (_Float16)val;
    } else {
        reinterpret_cast<uint16_t*>(a.o)[off] = (uint16_t)f32_to_bf16_bits(val);
    }
}

// Four consecutive head dims of one output row (element offset off, 4-aligned).
__device__ __forceinline__ void store_out4(const AttnArgs& a, int64_t off, f32x4 o) {
    if (a.out_kind == kOutF32) {
        *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(a.o) + off) = o;
    } else {
        const uint2 pk = a.out_kind == kOutF16 ? uint2{pack_f16x2_rn(o[0], o[1]), pack_f16x2_rn(o[2], o[3])}
                                               : uint2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.o) + off) = pk;
    }
}

// 16-bit input element type of the MFMA kernels: bf16 (F16 = false) or fp16.
template <bool F16> struct In16 { typedef bf16x8 v8; };
template <> struct In16<true> { typedef f16x8 v8; };

template <bool F16>
__device__ __forceinline__ f32x4 mfma_in(typename In16<F16>::v8 a, typename In16<F16>::v8 b, f32x4 c) {
    if constexpr (F16) return mfma16x16x32_f16(a, b, c);
    else return mfma16x16x32(a, b, c);
}

// p as an fp16 (hi, lo) pair, two weights per 32-bit word: hi = fp16(p),
// lo = fp16(p - hi) (~22 significant bits of p for p >= 2^-14).
__device__ __forceinline__ void split_f16x2(float p0, float p1, uint32_t& hi, uint32_t& lo) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 hv = __builtin_convertvector(f32x2v{p0, p1}, h2);
    const f32x2v hf = __builtin_convertvector(hv, f32x2v);
    const h2 lv = __builtin_convertvector(f32x2v{p0 - hf[0], p1 - hf[1]}, h2);
    hi = __builtin_bit_cast(uint32_t, hv);
    lo = __builtin_bit_cast(uint32_t, lv);
}

// ds_read_b64_tr_b16: within each 16-lane group, lane j receives element
// j%4 of the 8-byte rows addressed by lanes 4k + j/4, k = 0..3.  Lane i of a
// group addressing V[k0 + i/4][d0 + 4(i%4)] therefore gives lane j the four
// keys k0..k0+3 of head dim d0 + j: a V^T operand fragment read from V in
// its natural [key][d] layout.
typedef short v4i16 __attribute__((__vector_size__(8)));

__device__ __forceinline__ uint2 lds_read_tr16(const uint16_t* p) {
    const v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4i16*)(p));
    return __builtin_bit_cast(uint2, v);
}

typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));

// LDS reads of the ring kernel are written as asm: the compiler treats the
// builtin and plain forms as possible aliases of buffer_load ... lds writes
// still in flight and puts an s_waitcnt vmcnt(0) in front of them, which
// would wait for the NEXT tile's loads before the current tile is
// contracted (the caller has already waited for the stage it reads).  The
// asm reads do not wait: an explicit s_waitcnt asm that names them ties the wait for a batch of
// them to their result registers, so no use can be scheduled before it.
// Early-clobber outputs: a result register must not double as an address
// that a later read of the batch still has to send.
// OFF: a constant byte offset added to every address (the ring stage).
#define SF_TR16_X8(OFF)                                                                         \
    asm volatile("ds_read_b64_tr_b16 %0, %8 offset:" #OFF "\n\t"                              \
                 "ds_read_b64_tr_b16 %1, %9 offset:" #OFF "\n\t"                              \
                 "ds_read_b64_tr_b16 %2, %10 offset:" #OFF "\n\t"                             \
                 "ds_read_b64_tr_b16 %3, %11 offset:" #OFF "\n\t"                             \
                 "ds_read_b64_tr_b16 %4, %12 offset:" #OFF "\n\t"                             \
                 "ds_read_b64_tr_b16 %5, %13 offset:" #OFF "\n\t"                             \
                 "ds_read_b64_tr_b16 %6, %14 offset:" #OFF "\n\t"                             \
                 "ds_read_b64_tr_b16 %7, %15 offset:" #OFF                                     \
                 : "=&v"(o[0]), "=&v"(o[1]), "=&v"(o[2]), "=&v"(o[3]), "=&v"(o[4]), "=&v"(o[5]), \
                   "=&v"(o[6]), "=&v"(o[7])                                                    \
                 : "v"(addr[0]), "v"(addr[1]), "v"(addr[2]), "v"(addr[3]), "v"(addr[4]),       \
                   "v"(addr[5]), "v"(addr[6]), "v"(addr[7])                                    \
                 : "memory")
template <int OFF>
__device__ __forceinline__ void lds_read_tr16_x8(u32x2v (&o)[8], const uint32_t (&addr)[8]) {
    static_assert(OFF == 0 || OFF == 32768, "stage offsets of the ring");
    if constexpr (OFF == 0) SF_TR16_X8(0);
    else SF_TR16_X8(32768);
}
#undef SF_TR16_X8

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const char*)(p);
}

// Four ds_read_b128 (the wave's K fragments of a ring stage), no wait.
#define SF_B128_X4(OFF)                                                            \
    asm volatile("ds_read_b128 %0, %4 offset:" #OFF "\n\t"                       \
                 "ds_read_b128 %1, %5 offset:" #OFF "\n\t"                       \
                 "ds_read_b128 %2, %6 offset:" #OFF "\n\t"                       \
                 "ds_read_b128 %3, %7 offset:" #OFF                                \
                 : "=&v"(o[0]), "=&v"(o[1]), "=&v"(o[2]), "=&v"(o[3])             \
                 : "v"(addr[0]), "v"(addr[1]), "v"(addr[2]), "v"(addr[3])         \
                 : "memory")
template <int OFF>
__device__ __forceinline__ void lds_read_b128_x4(u32x4 (&o)[4], const uint32_t (&addr)[4]) {
    static_assert(OFF == 0 || OFF == 32768, "stage offsets of the ring");
    if constexpr (OFF == 0) SF_B128_X4(0);
    else SF_B128_X4(32768);
}
#undef SF_B128_X4

// max(x, x of lane ^ 16) and max(x, x of lane ^ 32) with the VALU lane swaps
// of gfx950 (v_permlane16/32_swap with both operands x: the two results hold,
// per lane, x of this row and of the partner row).  A ds_bpermute here would
// be an LDS instruction, in front of which the compiler also waits for the
// ring's in-flight DMA.
__device__ __forceinline__ float max_xor16(float x) {
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}

// x of lane l plus x of lane l ^ 16 (l ^ 32): lanes l, l ^ 16, l ^ 32 and
// l ^ 48 hold the four 8-element pieces of one MFMA operand row per register.
__device__ __forceinline__ float sum_xor16(float x) {
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

// Per-head RMSNorm of one bf16 row held as an MFMA operand (lane 16g + r:
// head dims 8g..8g+7 in f[0], 32+8g..32+8g+7 in f[1]), times gamma
// (gm[hh][0..1]: gamma[32hh + 8g ..+7]), rounded to bf16 in place -- the
// reference's rms_norm over head_dim (norm.cuh:89-122).  The arithmetic and
// the summation order are those of sf_gemm's per-head epilogue over a bf16
// product (heads16_kernel): each lane's eight squares in dim order, then
// the row's eight partial sums as ((s0 + s1) + (s2 + s3)) + ((s4 + s5) +
// (s6 + s7)), so the result is bit-identical to that epilogue's.
//
// norm_row16 is the general form: the row's 16-bit elements are read as
// bf16 or fp16 (IF16), normalised when `norm` (else only converted) and
// rounded to bf16 or fp16 (OF16).  fp16 rows are the projections' fp16
// outputs at large batch; the fp16 result feeds the fp16 MFMAs, the bf16
// one the bf16 MFMAs (a Q row against a bf16 K/V cache).
__device__ __forceinline__ float half_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

template <bool IF16, bool OF16>
__device__ __forceinline__ void norm_row16(u32x4 (&f)[2], const f32x4 (&gm)[2][2], bool norm, float eps) {
    float v[2][8];
    float part[2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        const u32x4 w = f[hh];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[hh][2 * e] = IF16 ? half_bits_to_f32(w[e] & 0xffffu) : bf16_bits_to_f32(w[e] & 0xffffu);
            v[hh][2 * e + 1] = IF16 ? half_bits_to_f32(w[e] >> 16) : bf16_bits_to_f32(w[e] >> 16);
        }
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) ss += v[hh][j] * v[hh][j];
        part[hh] = norm ? sum_xor32(sum_xor16(ss)) : 0.f;
    }
    const float inv_rms = 1.f / sqrtf((part[0] + part[1]) / 64.f + eps);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        u32x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const f32x4 g4 = gm[hh][e >> 1];
            const float x0 = norm ? v[hh][2 * e] * inv_rms * g4[(2 * e) & 3] : v[hh][2 * e];
            const float x1 = norm ? v[hh][2 * e + 1] * inv_rms * g4[(2 * e + 1) & 3] : v[hh][2 * e + 1];
            w[e] = OF16 ? pack_f16x2_rn(x0, x1) : pack_bf16x2(x0, x1);
        }
        f[hh] = w;
    }
}

__device__ __forceinline__ void rms_norm_row_bf16(bf16x8 (&f)[2], const f32x4 (&gm)[2][2], float eps) {
    u32x4 u[2] = {__builtin_bit_cast(u32x4, f[0]), __builtin_bit_cast(u32x4, f[1])};
    norm_row16<false, false>(u, gm, true, eps);
    f[0] = u32x4_as_bf16x8(u[0]);
    f[1] = u32x4_as_bf16x8(u[1]);
}

// The same on an fp16 operand row (normalised in fp32, rounded to fp16).
__device__ __forceinline__ void rms_norm_row_f16(f16x8 (&f)[2], const f32x4 (&gm)[2][2], float eps) {
    u32x4 u[2] = {__builtin_bit_cast(u32x4, f[0]), __builtin_bit_cast(u32x4, f[1])};
    norm_row16<true, true>(u, gm, true, eps);
    f[0] = u32x4_as_f16x8(u[0]);
    f[1] = u32x4_as_f16x8(u[1]);
}

// fp16 Q rows held in a bf16 operand: optionally normalised, rounded to bf16.
__device__ __forceinline__ void q_rows_f16_to_bf16(bf16x8 (&f)[2], const f32x4 (&gm)[2][2], bool norm, float eps) {
    u32x4 u[2] = {__builtin_bit_cast(u32x4, f[0]), __builtin_bit_cast(u32x4, f[1])};
    norm_row16<true, false>(u, gm, norm, eps);
    f[0] = u32x4_as_bf16x8(u[0]);
    f[1] = u32x4_as_bf16x8(u[1]);
}

// Either operand type: the per-head norm of a row of the kernel's own type.
__device__ __forceinline__ void rms_norm_row(bf16x8 (&f)[2], const f32x4 (&gm)[2][2], float eps) {
    rms_norm_row_bf16(f, gm, eps);
}
__device__ __forceinline__ void rms_norm_row(f16x8 (&f)[2], const f32x4 (&gm)[2][2], float eps) {
    rms_norm_row_f16(f, gm, eps);
}

// The eight gamma values of each of a lane's two operand pieces (zeros for
// a null gamma: a zero-range buffer reads zeros).
__device__ __forceinline__ void load_norm_gamma(const float* gamma, int g, f32x4 (&gm)[2][2]) {
    const __amdgpu_buffer_rsrc_t grs = make_rsrc(gamma, gamma ? 64u * 4u : 0u);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int i = 0; i < 2; ++i)
            gm[hh][i] = __builtin_bit_cast(f32x4, buffer_load16(grs, (uint32_t)((32 * hh + 8 * g + 4 * i) * 4)));
}

// Epilogue of the ring kernel: the four waves' (m, l, O) merged through LDS
// (xo_base: >= 64 KB of LDS no longer in use), then the normalised output
// (one split) or the split's partials.  Wave W owns head dims
// [16W, 16W + 16).  Every wave writes its row maxima and sums (lanes 0..15
// hold a row's sum in element 0 of the row-sum accumulator) and, unscaled,
// the three d-blocks it does not own; after
// ONE barrier each owner takes the four waves' maxima, scales the four
// contributions to its d-block and sums them, so each output element is
// summed once and stored as a 4-vector.  W is a template parameter (the
// caller switches on the wave index): the owner's block is then a constant
// register index, and every LDS read of the merge is issued before the
// first one is used (one LDS round trip instead of one per row block).
template <int W, int QB>
__device__ __forceinline__ void attn_split_epilogue(const AttnArgs& a, float* xo_base,
                                                    const f32x4 (&acc)[QB][4], const f32x4 (&accl)[QB],
                                                    const float (&m)[QB], int g, int r, int lane, int b,
                                                    int h, int q0, int split, int nsplit) {
    constexpr int QR = 16 * QB;
    float* xo = xo_base;                                  // [4 writer][3 slot][QB][64 lanes][4]
    float* sm = xo + 4 * 3 * QB * 64 * 4;                // [QR][4 writer]
    float* sl = sm + 4 * QR;                              // [QR][4 writer]
    static_assert((4 * 3 * QB * 64 * 4 + 2 * 4 * QR) * 4 <= 2 * 32768, "fits the ring's LDS");
#pragma unroll
    for (int o = 0; o < 4; ++o) {
        if (o == W) continue;
        const int slot = o - (o > W ? 1 : 0);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
            *reinterpret_cast<f32x4*>(xo + (((W * 3 + slot) * QB + qb) * 64 + lane) * 4) = acc[qb][o];
    }
    if (g == 0) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            sm[(16 * qb + r) * 4 + W] = m[qb];
            sl[(16 * qb + r) * 4 + W] = accl[qb][0];
        }
    }
    __syncthreads();

    // every read, then the arithmetic
    f32x4 mk[QB], lk[QB], c[QB][3];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        mk[qb] = *reinterpret_cast<const f32x4*>(sm + (16 * qb + r) * 4);
        lk[qb] = *reinterpret_cast<const f32x4*>(sl + (16 * qb + r) * 4);
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int k = j + (j >= W ? 1 : 0);          // the other writers, in wave order
            const int slot = W - (W > k ? 1 : 0);        // W's slot in writer k's blocks
            c[qb][j] = *reinterpret_cast<const f32x4*>(xo + (((k * 3 + slot) * QB + qb) * 64 + lane) * 4);
        }
    }
    const size_t bh = (size_t)b * a.H + h;
    const size_t pbase = (bh * nsplit + split) * (size_t)a.Sq;
    const int d0 = 16 * W + 4 * g;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        const float M = fmaxf(fmaxf(mk[qb][0], mk[qb][1]), fmaxf(mk[qb][2], mk[qb][3]));
        const float Muse = M == -INFINITY ? 0.f : M;
        float f[4];
        float L = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            f[k] = fast_exp2(mk[qb][k] - Muse);
            L += lk[qb][k] * f[k];
        }
        f32x4 o = acc[qb][W] * f[W];
#pragma unroll
        for (int j = 0; j < 3; ++j) o += c[qb][j] * f[j + (j >= W ? 1 : 0)];
        const int q = q0 + 16 * qb + r;
        if (q >= a.Sq) continue;
        if (nsplit == 1) {
            o *= L > 0.f ? __builtin_amdgcn_rcpf(L) : 0.f;
            store_out4(a, b * a.o_sb + h * a.o_sh + q * a.o_ss + d0, o);
        } else {
            // non-temporal: the merge kernel reads the partials once, and
            // stores that do not linger dirty in L2 leave less to write back
            // at the kernel boundary (batch-1 image op 15.7 -> 14.6 us)
            __builtin_nontemporal_store(o, reinterpret_cast<f32x4*>(a.part_o + (pbase + q) * kD + d0));
            if (W == 0 && g == 0) {
                __builtin_nontemporal_store(M, a.part_ml + (pbase + q) * 2);
                __builtin_nontemporal_store(L, a.part_ml + (pbase + q) * 2 + 1);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Split kernel, ring-pipelined (the cross-attention path).
//
// One (b, h, query chunk, key split) per workgroup of 4 waves; two
// workgroups fit on a CU (64 KB of LDS each), and the split count puts about
// one per CU (choose_splits).  K and V tiles of 128 keys go HBM -> LDS directly
// (buffer_load ... lds, no VGPR staging) into a 2-stage ring per workgroup,
// a tile's loads issued as soon as its stage is free.  Rows
// sit in LDS in their natural [key][64] layout with the 16-byte chunks of
// key row k XOR-swizzled by (k >> 1) & 7, which makes both the K fragment
// reads (16 rows x 16 B) and the V^T transpose reads (4 rows x 8 B per
// 16-lane group) bank-conflict free.  Q fragments live in registers.  The
// arithmetic: S^T = K.Q^T, lazy-rescaled log2 softmax, O^T += V^T.P^T
// (fp16, or bf16 with P as a hi/lo pair), 4-wave LDS merge; the row sums
// come from the MFMA pipe: a constant V^T fragment whose first row is all
// ones turns P^T into l, so the VALU does no per-element adds and l sums
// exactly the rounded weights the numerator uses.
// ---------------------------------------------------------------------------
constexpr int kRingStages = 2;
constexpr int kKT = 128;                          // keys per tile (4 waves x 32)
constexpr int kTileBytes = kKT * kD * 2;          // 16 KB per K (or V) tile
constexpr int kStageBytes = 2 * kTileBytes;       // K then V

__device__ __forceinline__ int ring_swz(int key) { return (key >> 1) & 7; }

// Cache policy of the K/V tile loads: nt (non-temporal), since every K/V
// byte is read once per call.  A plain streaming read of a cold 1 GiB
// buffer on MI355X moves 7.1 TB/s with nt against 6.2 TB/s without.
constexpr int kKvPolicy = 2;

template <int V> struct StageOff { static constexpr int value = V; };

// Key-padding mask bytes of keys k..k+3 (k a multiple of 4) as a 32-bit
// word.  The buffer range is Sk rounded up to 4 bytes: words past it read as
// 0, and bytes of keys >= Sk are never used (those keys are out of range).
__device__ __forceinline__ uint32_t mask_word(__amdgpu_buffer_rsrc_t mrs, int key) {
    return __builtin_amdgcn_raw_buffer_load_b32(mrs, (uint32_t)key, 0, 0);
}

// Wait until at most one tile's loads (8 per wave) of this wave are still
// outstanding: the older tile has landed.  Vector loads complete in issue
// order, so this covers the tile being waited for and every load issued
// before it (Q, mask words).  No barrier: a wave's DMA fills exactly the 32
// key rows of K and V that the same wave contracts, so no wave ever reads
// LDS that another wave writes inside the tile loop.
__device__ __forceinline__ void ring_wait() {
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
}

// Wait for the K half of the older tile only (issued before its V half, so
// at most V of that tile and the 8 loads of the next tile are outstanding).
__device__ __forceinline__ void ring_wait_k() {
    asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
}

// kExactPV false: P.V in fp16 with P rounded to fp16 (a bf16 V converted,
// exact for 2^-14 <= |v| < 2^16; an fp16 V as is).  true: V in its input
// type and P as a (hi, lo) pair of that type.  kF16: Q/K/V are fp16 (S on
// the fp16 MFMA) instead of bf16.  QB: 16-row query blocks per workgroup
// (kQB on the (split x chunk, H, B) grid; 1 on the XCD-grouped 1-D grid).
// kQP (QB = 1, bf16): Q is finished here from its projection's split-K
// partials (sum, scale, bias, per-head RMSNorm, bf16) instead of loaded.
// kVH (bf16 Q/K, fp16 form): V is given in fp16 and used as loaded.
template <bool kExactPV, bool kF16, int QB, bool kQP = false, bool kVH = false>
__global__ __launch_bounds__(256, 2) void attn_ring_kernel(const AttnArgs a) {
    static_assert(!(kVH && (kExactPV || kF16)), "fp16 V: the fp16 P.V form of bf16 Q/K");
    using v8 = typename In16<kF16>::v8;
    constexpr int QR = 16 * QB;
    __shared__ __attribute__((aligned(16))) char ring[kRingStages * kStageBytes];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // the wave index as a scalar, so the LDS-DMA destinations (M0) and the
    // per-tile buffer resources are scalar arithmetic
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4;
    const int r = lane & 15;
    const int nsplit = a.nsplit;
    int split, qc, h, b;
    if constexpr (QB == 1) {
        // 1-D grid of one 16-row query block per workgroup, no key split:
        // id = slot + 8 (chunk + nqc * head group), so the blocks of head
        // 8 group + slot sit at ids congruent mod 8, on one XCD, and its K/V
        // are fetched into that L2 once and read from there by every block.
        const int id = blockIdx.x;
        const int rest = id >> 3;
        const int bh = (id & 7) + 8 * (rest / a.nqc);
        if (bh >= a.B * a.H) return;   // the grid's last head group is padded to 8
        qc = rest % a.nqc;
        h = bh % a.H;
        b = bh / a.H;
        split = 0;
    } else {
        split = blockIdx.x % nsplit;
        qc = blockIdx.x / nsplit;
        h = blockIdx.y;
        b = blockIdx.z;
    }
    const int q0 = qc * QR;

    int valid = a.Sk;
    if (a.valid_len) {
        const int vl = a.valid_len[b];
        valid = vl < 0 ? 0 : (vl > a.Sk ? a.Sk : vl);
    }
    // Key range of this split: equal shares of the VALID keys, 32-key granular.
    int per = (valid + nsplit - 1) / nsplit;
    per = (per + 31) & ~31;
    const int kbeg = split * per;
    int kend = min(valid, kbeg + per);
    if (a.causal) kend = min(kend, min(a.Sq, q0 + QR));
    const int ntiles = kend > kbeg ? (kend - kbeg + kKT - 1) / kKT : 0;

    const uint16_t* qp = a.q + b * a.q_sb + h * a.q_sh;
    const uint16_t* kp = a.k + b * a.k_sb + h * a.k_sh;
    const uint16_t* vp = a.v + b * a.v_sb + h * a.v_sh;
    const __amdgpu_buffer_rsrc_t qrs = make_rsrc(qp, (uint32_t)(a.Sq * a.q_ss * 2));
    const __amdgpu_buffer_rsrc_t mrs =
        make_rsrc(a.kv_mask ? static_cast<const void*>(a.kv_mask + b * a.kv_mask_stride) : static_cast<const void*>(a.q),
                  a.kv_mask ? (uint32_t)((a.Sk + 3) & ~3) : 0u);

    // Q fragments (B operand of S^T = K.Q^T): row 16qb + r, dims 32hh + 8g..
    v8 qf[QB][2];
    // kQP: wave w finishes rows q0 + 4w .. q0 + 4w + 3, lane l row
    // q0 + 4w + l/16 and dims 4(l%16) .. +3 -- the reduce_heads epilogue's
    // layout and arithmetic, so Q is bit-identical to the unfused path.
    // Every split's loads go out here, before the ring's first tiles; rows
    // past Sq and splits past q_splits read as zeros.
    constexpr int kQPMax = 8;
    f32x4 qpv[kQP ? kQPMax : 1];
    f32x4 qbias, qscale, qgam;
    float qrss[4] = {0.f, 0.f, 0.f, 0.f};
    if constexpr (kQP) {
        static_assert(QB == 1 && !kF16, "Q from partials: the bf16 query-block instance");
        const int row = q0 + 4 * w + (lane >> 4);
        const int c4 = 4 * (lane & 15);
        const bool rlive = row < a.Sq;
        const uint32_t rowoff = rlive ? (uint32_t)(((int64_t)b * a.Sq + row) * (a.H * 64) + h * 64 + c4) : 0u;
        const uint32_t sstride = (uint32_t)((int64_t)a.B * a.Sq * a.H * 64);
        const __amdgpu_buffer_rsrc_t prs = make_rsrc(a.qp, a.qp_bytes);
#pragma unroll
        for (int j = 0; j < kQPMax; ++j) {
            const uint32_t off = j < a.q_splits && rlive ? (rowoff + j * sstride) * 4u
                                                         : 0x80000000u;   // past the buffer range: zeros
            qpv[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(prs, off, 0, kKvPolicy));
        }
        const int nb = h * 64 + c4;
        const __amdgpu_buffer_rsrc_t brs = make_rsrc(a.q_bias, a.q_bias ? (uint32_t)(a.H * 64 * 4) : 0u);
        const __amdgpu_buffer_rsrc_t srs = make_rsrc(a.q_scale, a.q_scale ? (uint32_t)(a.H * 64 * 4) : 0u);
        const __amdgpu_buffer_rsrc_t grs = make_rsrc(a.q_gamma, a.q_gamma ? 64u * 4u : 0u);
        qbias = __builtin_bit_cast(f32x4, buffer_load16(brs, (uint32_t)(nb * 4)));
        qscale = __builtin_bit_cast(f32x4, buffer_load16(srs, (uint32_t)(nb * 4)));
        qgam = __builtin_bit_cast(f32x4, buffer_load16(grs, (uint32_t)(c4 * 4)));
        if (a.q_row_ss) {   // the deferred norm's tile sums of this lane's row
            const int64_t prow = (int64_t)b * a.Sq + (rlive ? row : 0);
            const int64_t M = (int64_t)a.B * a.Sq;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int t = (lane & 15) + 16 * k;
                qrss[k] = t < a.q_row_tiles ? a.q_row_ss[t * M + prow] : 0.f;
            }
        }
    } else {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
                qf[qb][hh] = __builtin_bit_cast(
                    v8, buffer_load16(qrs, (uint32_t)(((q0 + 16 * qb + r) * a.q_ss + 32 * hh + 8 * g) * 2)));
    }
    // q_norm weight for Q rows normalised as they are loaded (bf16)
    f32x4 qgm[2][2];
    if constexpr (!kQP) load_norm_gamma(a.q_gamma, g, qgm);

    // DMA of one tile into a stage: wave w, op j fills LDS chunks
    // (4w + j) * 64 + lane = key * 8 + slot of K (and of V), loading global
    // chunk slot ^ swz(key) of that key.  The tile's rows are addressed
    // through a buffer resource based at the tile's first key and ending at
    // kend (scalar work per tile), so the per-lane offsets are the same for
    // every tile and keys past kend read as zeros.
    uint32_t koffj[4], voffj[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int p = (4 * w + j) * 64 + lane;
        const int key = p >> 3;
        const int col = ((p & 7) ^ ring_swz(key)) * 8;
        koffj[j] = (uint32_t)((key * a.k_ss + col) * 2);
        voffj[j] = (uint32_t)((key * a.v_ss + col) * 2);
    }
    auto issue = [&](int t) {
        const int kt = kbeg + t * kKT;
        const uint32_t rows = (uint32_t)max(kend - kt, 0);
        const __amdgpu_buffer_rsrc_t krs = make_rsrc(kp + (int64_t)kt * a.k_ss, rows * (uint32_t)a.k_ss * 2u);
        const __amdgpu_buffer_rsrc_t vrs = make_rsrc(vp + (int64_t)kt * a.v_ss, rows * (uint32_t)a.v_ss * 2u);
        char* st = ring + (t % kRingStages) * kStageBytes;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                krs, (__attribute__((address_space(3))) void*)(st + (4 * w + j) * 1024), 16, koffj[j], 0, 0,
                kKvPolicy);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                vrs, (__attribute__((address_space(3))) void*)(st + kTileBytes + (4 * w + j) * 1024), 16,
                voffj[j], 0, 0, kKvPolicy);
    };
    // Key-padding mask words of tile t, loaded one tile ahead and always
    // BEFORE the next tile's DMA is issued: vector loads complete in issue
    // order, so the wait the compiler puts in front of their first use then
    // never covers a tile still streaming in.
    auto load_mask = [&](int t, uint32_t (&mw)[2]) {
        const int kt = kbeg + t * kKT;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) mw[kb] = mask_word(mrs, kt + 32 * w + 16 * kb + 4 * g);
    };
    uint32_t mw_next[2] = {0xffffffffu, 0xffffffffu};
    if (a.kv_mask) load_mask(0, mw_next);
    // Exactly one tile is issued per stage use, whether or not it exists:
    // tiles at or past ntiles lie beyond the buffer range and load zeros (no
    // memory traffic).  With the issue unconditional, the compiler's own
    // vmcnt bookkeeping sees the ring loads as always in flight behind Q and
    // the mask words, and ring_wait waits for one tile at a time.
    issue(0);
    issue(1);
    if constexpr (kQP) {
        // Q = rmsnorm_64(sum_j part_j * scale + bias) * gamma in bf16, as
        // reduce_heads_kernel computes it (slices summed in ascending order;
        // no scale = 1, no bias = 0, no gamma = no norm), rows exchanged
        // through LDS so that every wave holds the fragments of all 16.  The
        // LDS accesses are inline asm: the compiler would otherwise wait for
        // the in-flight ring DMA in front of them.
        __shared__ __attribute__((aligned(16))) uint16_t qlds[16 * 64];
        f32x4 v = qpv[0];
#pragma unroll
        for (int j = 1; j < kQPMax; ++j)
            if (j < a.q_splits) v += qpv[j];
        if (a.q_row_ss) {   // as reduce_heads_kernel over x * gamma rows (deferred_row_scale)
            float tsum = 0.f;
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if ((lane & 15) + 16 * k < a.q_row_tiles) tsum += qrss[k];
            const float rs = deferred_rsqrt(row16_sum(tsum), a.q_row_inv_n, a.q_row_eps);
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = deferred_affine(v[i], a.q_scale ? qscale[i] : 1.f, rs, qbias[i]);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = v[i] * (a.q_scale ? qscale[i] : 1.f) + qbias[i];
        }
        if (a.q_gamma) {
            float ss = v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
            ss = row16_sum(ss);
            const float inv_rms = 1.f / sqrtf(ss / 64.f + a.q_eps);
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = v[i] * inv_rms * qgam[i];
        }
        const uint32_t qbase = lds_addr(qlds);
        const uint32_t waddr = qbase + (uint32_t)(((4 * w + (lane >> 4)) * 64 + 4 * (lane & 15)) * 2);
        const uint32_t wlo = pack_bf16x2(v[0], v[1]), whi = pack_bf16x2(v[2], v[3]);
        asm volatile("ds_write_b64 %0, %1\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier"
                     :: "v"(waddr), "v"(uint2{wlo, whi}) : "memory");
        u32x4 q0w, q1w;
        const uint32_t raddr = qbase + (uint32_t)((r * 64 + 8 * g) * 2);
        asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %2 offset:64\n\ts_waitcnt lgkmcnt(0)"
                     : "=&v"(q0w), "=&v"(q1w) : "v"(raddr) : "memory");
        qf[0][0] = __builtin_bit_cast(v8, q0w);
        qf[0][1] = __builtin_bit_cast(v8, q1w);
    }
    // Wait for the Q fragments here, behind the first tiles' loads.  Inside
    // the tile loop the compiler would otherwise still count them as
    // outstanding and wait for every in-flight ring load before the first
    // S contraction of each tile.
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) asm volatile("" ::"v"(qf[qb][hh]));
    if constexpr (!kQP) {
        if constexpr (!kF16) {
            if (a.q_f16) {   // fp16 rows: normalised (with q_gamma) and rounded to bf16
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) q_rows_f16_to_bf16(qf[qb], qgm, a.q_gamma != nullptr, a.q_eps);
            } else if (a.q_gamma) {
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) rms_norm_row_bf16(qf[qb], qgm, a.q_eps);
            }
        } else if (a.q_gamma) {
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) rms_norm_row_f16(qf[qb], qgm, a.q_eps);
        }
    }

    f32x4 acc[QB][4];   // O^T blocks: lane holds d = 16db + 4g + i, q = 16qb + r
    f32x4 accl[QB];     // row sums: element 0 of lanes 0..15 holds l of query 16qb + r
    // m: running max of each query row in log2 units (-inf until a finite
    // score has been seen); nm: the offset the weights use, -m (0 while m is
    // -inf).  A tile whose raw scores stay at or below (m + 8) / scale_log2
    // keeps m, so every weight is <= 2^8.
    float m[QB], nm[QB];
    const float inv_sl2 = 1.f / a.scale_log2;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        m[qb] = -INFINITY;
        nm[qb] = 0.f;
        accl[qb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int db = 0; db < 4; ++db) acc[qb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    // A operand whose row 0 is all ones (rows 1..15 zero)
    const uint32_t one2 = r == 0 ? 0x3f803f80u : 0u;
    const bf16x8 ones = u32x4_as_bf16x8(u32x4{one2, one2, one2, one2});
    const uint32_t oneh = r == 0 ? 0x3c003c00u : 0u;
    const f16x8 ones_f16 = u32x4_as_f16x8(u32x4{oneh, oneh, oneh, oneh});

    const int wkey = 32 * w;   // this wave's first key inside a tile
    // LDS byte addresses of this lane's K fragment and V^T transpose reads in
    // stage 0 (swizzled rows); stage 1 adds the reads' constant offset field
    static_assert(kStageBytes == 32768 && kRingStages == 2, "the LDS reads encode the stage offset");
    const uint32_t lbase = lds_addr(ring);
    uint32_t ka[4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
        const int key = wkey + 16 * kb + r;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) ka[2 * kb + hh] = lbase + key * 128 + (((g + 4 * hh) ^ ring_swz(key)) * 16);
    }
    uint32_t va[8];   // [2 db + key half]
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
        const int key = wkey + 16 * hf + 4 * g + (r >> 2);
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            const int d = 16 * db + 4 * (r & 3);
            va[2 * db + hf] = lbase + kTileBytes + key * 128 + (((d >> 3) ^ ring_swz(key)) * 16) + (d & 7) * 2;
        }
    }

    // One tile; SOFF (0 or kStageBytes) is the stage it sits in, t % 2.
    auto tile = [&](const int t, auto soff) {
        constexpr int SOFF = decltype(soff)::value;
        const int kt = kbeg + t * kKT;
        // Tile t's K has landed (tile t's V and tile t + 1 may still stream
        // in); with a key-padding mask the mask words of tile t sit behind
        // its V in the load queue, so the whole tile is waited for.
        if (a.kv_mask) ring_wait();
        else ring_wait_k();
        if (kt + wkey < kend && !(a.causal && kt + wkey > q0 + QR - 1)) {
            // K fragments for the S contraction; V is waited for and read
            // (V^T) only after S and the softmax statistics, so its DMA
            // overlaps them and its transpose reads overlap the weights.
            u32x4 kw[4];
            lds_read_b128_x4<SOFF>(kw, ka);
            // K landed (LDS reads return in order; no scalar loads are in
            // flight in the loop, so the count is exact)
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(kw[0]), "+v"(kw[1]), "+v"(kw[2]), "+v"(kw[3]) :: "memory");
            v8 kf[2][2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) kf[kb][hh] = __builtin_bit_cast(v8, kw[2 * kb + hh]);
            const bool need_mask = a.causal || kt + kKT > kend || a.kv_mask;
            const uint32_t mw[2] = {mw_next[0], mw_next[1]};
            f32x4 s[QB][2];
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    f32x4 z = {0.f, 0.f, 0.f, 0.f};
                    z = mfma_in<kF16>(kf[kb][0], qf[qb][0], z);
                    s[qb][kb] = mfma_in<kF16>(kf[kb][1], qf[qb][1], z);
                }
            }
            if (need_mask) {
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) {
                    const int qrow = q0 + 16 * qb + r;
#pragma unroll
                    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int key = kt + wkey + 16 * kb + 4 * g + i;
                            const bool dead = key >= kend || (a.causal && key > qrow) ||
                                              ((mw[kb] >> (8 * i)) & 0xffu) == 0;
                            s[qb][kb][i] = dead ? -INFINITY : s[qb][kb][i];
                        }
                    }
                }
            }
            // The lane's own maximum over its 8 scores of each row block.  A
            // row's maximum over the tile exceeds its threshold exactly when
            // one of the four lanes holding that row does, so the wave-wide
            // test needs no cross-lane maximum; that is taken only when the
            // rows are rescaled.
            float lmx[QB];
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                const f32x4 u = s[qb][0], v = s[qb][1];
                lmx[qb] = fmaxf(fmaxf(fmaxf(fmaxf(fmaxf(fmaxf(fmaxf(u[0], u[1]), u[2]), u[3]), v[0]), v[1]), v[2]),
                                v[3]);
            }
            bool grow = false;
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) grow |= lmx[qb] > fmaf(m[qb], inv_sl2, 8.f * inv_sl2);
            if (__any(grow)) {
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) {
                    const float mx = max_xor32(max_xor16(lmx[qb])) * a.scale_log2;
                    const float mnew = fmaxf(m[qb], mx);
                    if constexpr (!kExactPV) nm[qb] = mnew == -INFINITY ? 0.f : -mnew;
                    const float alpha = fast_exp2(m[qb] - (mnew == -INFINITY ? 0.f : mnew));
                    m[qb] = mnew;
                    accl[qb] *= alpha;
#pragma unroll
                    for (int db = 0; db < 4; ++db) acc[qb][db] *= alpha;
                }
            }
            // Tile t's V has landed; the transpose reads go out now and are
            // waited for after the weights of every row block are formed.
            ring_wait();
            u32x2v vt[8];
            lds_read_tr16_x8<SOFF>(vt, va);
            // Weights: P rounded to the nearest fp16 (P <= 2^8 by the lazy
            // rescale; l sums the same rounded weights), or a (hi, lo) pair
            // of the input type in the exact form.
            f16x8 p8[QB];
            bf16x8 ph8[QB], pl8[QB];
            f16x8 hh8[QB], hl8[QB];
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                if constexpr (!kExactPV) {
                    float pf[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) pf[j] = fast_exp2(fmaf(s[qb][j >> 2][j & 3], a.scale_log2, nm[qb]));
                    p8[qb] = u32x4_as_f16x8(u32x4{pack_f16x2_rn(pf[0], pf[1]), pack_f16x2_rn(pf[2], pf[3]),
                                                  pack_f16x2_rn(pf[4], pf[5]), pack_f16x2_rn(pf[6], pf[7])});
                } else if constexpr (kF16) {
                    const float nmuse = m[qb] == -INFINITY ? 0.f : -m[qb];
                    uint32_t hw[4], lw[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        split_f16x2(fast_exp2(fmaf(s[qb][(2 * e) >> 2][(2 * e) & 3], a.scale_log2, nmuse)),
                                    fast_exp2(fmaf(s[qb][(2 * e + 1) >> 2][(2 * e + 1) & 3], a.scale_log2, nmuse)),
                                    hw[e], lw[e]);
                    hh8[qb] = u32x4_as_f16x8(u32x4{hw[0], hw[1], hw[2], hw[3]});
                    hl8[qb] = u32x4_as_f16x8(u32x4{lw[0], lw[1], lw[2], lw[3]});
                } else {
                    const float nmuse = m[qb] == -INFINITY ? 0.f : -m[qb];
                    uint32_t pb[8], lb[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const float p = fast_exp2(fmaf(s[qb][j >> 2][j & 3], a.scale_log2, nmuse));
                        pb[j] = __float_as_uint(p);
                        lb[j] = __float_as_uint(p - __uint_as_float(pb[j] & 0xffff0000u));
                    }
                    ph8[qb] = u32x4_as_bf16x8(u32x4{__builtin_amdgcn_perm(pb[1], pb[0], 0x07060302u),
                                                    __builtin_amdgcn_perm(pb[3], pb[2], 0x07060302u),
                                                    __builtin_amdgcn_perm(pb[5], pb[4], 0x07060302u),
                                                    __builtin_amdgcn_perm(pb[7], pb[6], 0x07060302u)});
                    pl8[qb] = u32x4_as_bf16x8(u32x4{__builtin_amdgcn_perm(lb[1], lb[0], 0x07060302u),
                                                    __builtin_amdgcn_perm(lb[3], lb[2], 0x07060302u),
                                                    __builtin_amdgcn_perm(lb[5], lb[4], 0x07060302u),
                                                    __builtin_amdgcn_perm(lb[7], lb[6], 0x07060302u)});
                }
            }
            // V^T fragments: bf16 as read (exact form), or converted to fp16
            // with rounding to nearest, which is exact for 2^-14 <= |v| < 2^16
            // (bf16's 8 significant bits fit fp16's 11), within 2^-25 below
            // (fp16's subnormal grid) and gives +-inf above: an
            // out-of-range (or infinite or NaN) v makes the output columns it
            // reaches inf or NaN, never a saturated value.
            bf16x8 vf[4];
            f16x8 vh[4];
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(vt[0]), "+v"(vt[1]), "+v"(vt[2]), "+v"(vt[3]),
                         "+v"(vt[4]), "+v"(vt[5]), "+v"(vt[6]), "+v"(vt[7]) :: "memory");
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const u32x4 vw = {vt[2 * db][0], vt[2 * db][1], vt[2 * db + 1][0], vt[2 * db + 1][1]};
                if constexpr (kF16 || kVH) {
                    vh[db] = u32x4_as_f16x8(vw);   // fp16 V as loaded
                } else if constexpr (kExactPV) {
                    vf[db] = u32x4_as_bf16x8(vw);
                } else {
                    u32x4 hw;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float lo = __uint_as_float(vw[e] << 16);
                        const float hi = __uint_as_float(vw[e] & 0xffff0000u);
                        hw[e] = pack_f16x2_rn(lo, hi);
                    }
                    vh[db] = u32x4_as_f16x8(hw);
                }
            }
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                if constexpr (!kExactPV) {
#pragma unroll
                    for (int db = 0; db < 4; ++db) acc[qb][db] = mfma16x16x32_f16(vh[db], p8[qb], acc[qb][db]);
                    accl[qb] = mfma16x16x32_f16(ones_f16, p8[qb], accl[qb]);
                } else if constexpr (kF16) {
#pragma unroll
                    for (int db = 0; db < 4; ++db) {
                        acc[qb][db] = mfma16x16x32_f16(vh[db], hh8[qb], acc[qb][db]);
                        acc[qb][db] = mfma16x16x32_f16(vh[db], hl8[qb], acc[qb][db]);
                    }
                    accl[qb] = mfma16x16x32_f16(ones_f16, hh8[qb], accl[qb]);
                    accl[qb] = mfma16x16x32_f16(ones_f16, hl8[qb], accl[qb]);
                } else {
#pragma unroll
                    for (int db = 0; db < 4; ++db) {
                        acc[qb][db] = mfma16x16x32(vf[db], ph8[qb], acc[qb][db]);
                        acc[qb][db] = mfma16x16x32(vf[db], pl8[qb], acc[qb][db]);
                    }
                    accl[qb] = mfma16x16x32(ones, ph8[qb], accl[qb]);
                    accl[qb] = mfma16x16x32(ones, pl8[qb], accl[qb]);
                }
            }
        }   // live keys
        // this wave's reads of the stage are done before its rows are refilled
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (a.kv_mask) load_mask(t + 1, mw_next);
        issue(t + kRingStages);
    };
    // Two tiles per iteration, one per stage, so every LDS read of a tile
    // carries its stage as a constant offset.
    for (int t = 0; t < ntiles; t += 2) {
        tile(t, StageOff<0>{});
        if (t + 1 < ntiles) tile(t + 1, StageOff<kStageBytes>{});
    }
    // The loads issued past the last tile land in LDS that the epilogue
    // reuses: every wave waits for its own, then all waves meet.
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    float* xo = reinterpret_cast<float*>(ring);
    switch (w) {   // wave-uniform
        case 0: attn_split_epilogue<0, QB>(a, xo, acc, accl, m, g, r, lane, b, h, q0, split, nsplit); break;
        case 1: attn_split_epilogue<1, QB>(a, xo, acc, accl, m, g, r, lane, b, h, q0, split, nsplit); break;
        case 2: attn_split_epilogue<2, QB>(a, xo, acc, accl, m, g, r, lane, b, h, q0, split, nsplit); break;
        default: attn_split_epilogue<3, QB>(a, xo, acc, accl, m, g, r, lane, b, h, q0, split, nsplit); break;
    }
}

// Log-sum-exp merge of the split partials.  One wave per output row
// (b, h, q): lane s < nsplit loads split s's (max, sum) and every lane loads
// head dim d = lane of every split's partial output, all up front; the
// splits' (max, sum) then come to every lane through v_readlane (scalar
// registers, no LDS round trips), and each lane forms
// out = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s.
__global__ __launch_bounds__(256) void attn_merge_kernel(const AttnArgs a) {
    const int lane = threadIdx.x & 63;
    const int q = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int h = blockIdx.y;
    const int b = blockIdx.z;
    if (q >= a.Sq) return;
    const int ns = a.nsplit;   // <= kMaxSplits = 64
    const size_t row0 = ((size_t)b * a.H + h) * ns * (size_t)a.Sq + q;   // split 0's row
    constexpr int kMergeBatch = 16;
    float ms = -INFINITY, ls = 0.f;
    if (lane < ns) {
        const float2 ml = *reinterpret_cast<const float2*>(a.part_ml + (row0 + (size_t)lane * a.Sq) * 2);
        ms = ml.x;
        ls = ml.y;
    }
    float v0[kMergeBatch];
#pragma unroll
    for (int j = 0; j < kMergeBatch; ++j)
        if (j < ns) v0[j] = a.part_o[(row0 + (size_t)j * a.Sq) * kD + lane];
    float M = -INFINITY;
    for (int j = 0; j < ns; ++j) M = fmaxf(M, __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_int(ms), j)));
    const float Muse = M == -INFINITY ? 0.f : M;
    float L = 0.f, o = 0.f;
#pragma unroll
    for (int j = 0; j < kMergeBatch; ++j) {
        if (j < ns) {
            const float e = fast_exp2(__builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_int(ms), j)) - Muse);
            L += e * __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_int(ls), j));
            o += e * v0[j];
        }
    }
    for (int s0 = kMergeBatch; s0 < ns; s0 += 8) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            v[j] = s0 + j < ns ? a.part_o[(row0 + (size_t)(s0 + j) * a.Sq) * kD + lane] : 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (s0 + j < ns) {
                const float e = fast_exp2(
                    __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_int(ms), s0 + j)) - Muse);
                L += e * __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_int(ls), s0 + j));
                o += e * v[j];
            }
        }
    }
    o *= L > 0.f ? 1.f / L : 0.f;
    store_out(a, b, h, q, lane, o);
}

// ---------------------------------------------------------------------------
// Short key sets (Sk <= 128: the 67 x 67 self-attention of every block, short
// language conditions): one wave per (b, h, 16-query block), all of K, V and
// the query block loaded at once (one memory round trip), a single-pass
// softmax over the whole key set (no running max, no split, no cross-wave
// merge), and the result stored straight from the accumulators.
//
// S^T = K.Q^T with K fragments loaded from global directly in MFMA operand
// layout.  V is staged in LDS in its natural [key][d] layout and read back as
// the V^T operand with ds_read_b64_tr_b16: within each 16-lane group, lane j
// receives element j%4 of the 8-byte rows addressed by lanes 4k + j/4,
// k = 0..3, so lane i of group g addressing V[k0 + i/4][d0 + 4(i%4)] gives
// lane j the four keys k0..k0+3 of head dim d0 + j -- the V^T fragment whose
// key order matches the P^T slots the S^T accumulator provides.
// ---------------------------------------------------------------------------
constexpr int kShortMaxKeys = 128;
// B*H from which a workgroup takes all of a head's query blocks, one wave
// each, sharing one LDS copy of the head's K and V (27 KB at 67 keys).
// Same-box A/B, self-attention over the QKV rows with q/k norm on load,
// against one-wave workgroups: B=8 7.2 vs 8.6 us (per-wave V copies),
// B=16 12.5 vs 15.2, B=32 22.5 vs 23.3.  (With a V copy per wave, 77 KB per
// workgroup, the grouped form had lost at B*H = 1024: 20.9 vs 19.4 us.)
constexpr long kShortGroupMinHeads = 256;
constexpr int kVPitch = 80;   // LDS row pitch of V (bf16): 160 B keeps the four rows of a read apart

// NW query blocks per workgroup, one wave each: 1 spreads a small batch's
// few heads over the most CUs; 5 (large batches) runs a head's 67 queries on
// one CU, whose waves load K and V once between them.
// kVH: bf16 Q/K with fp16 V (P then an fp16 (hi, lo) pair, as for fp16 inputs).
template <int KB, bool kF16, int NW, bool kVH = false>   // 16-key blocks covering Sk (even, <= 8); fp16 (else bf16) Q/K/V
__global__ __launch_bounds__(64 * NW) void attn_short_kernel(const AttnArgs a) {
    static_assert(!(kVH && kF16), "fp16 V with bf16 Q/K");
    using v8 = typename In16<kF16>::v8;
    constexpr int KROWS = 16 * KB;
    // NW == 1: the wave loads all of K and V and stages V in LDS.  NW > 1:
    // the workgroup's waves share one V region and one region of K operand
    // fragments ([KB][64 lanes][2]): wave w loads every NW-th V chunk and the
    // K blocks kb = w, w + NW, ... (normalising them with k_gamma), all
    // waves meet at one barrier and then read every block -- one copy of K
    // and V per head, so more heads share a CU.  Every wave of a grouped
    // workgroup, even one past the queries, loads its share and meets the
    // barrier; a one-wave workgroup past the queries just ends.
    __shared__ __attribute__((aligned(16))) uint16_t vls[KROWS * kVPitch];
    __shared__ __attribute__((aligned(16))) u32x4 kls[NW > 1 ? KB * 64 * 2 : 1];
    const int lane = threadIdx.x & 63;
    const int w = NW > 1 ? __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6) : 0;
    uint16_t* vl = vls;
    const int g = lane >> 4;
    const int r = lane & 15;
    const int q0 = 16 * ((int)blockIdx.x * NW + w);
    if constexpr (NW == 1) {
        if (q0 >= a.Sq) return;
    }
    const int h = blockIdx.y;
    const int b = blockIdx.z;

    int valid = a.Sk;
    if (a.valid_len) {
        const int vl_ = a.valid_len[b];
        valid = vl_ < 0 ? 0 : (vl_ > a.Sk ? a.Sk : vl_);
    }
    const uint16_t* qp = a.q + b * a.q_sb + h * a.q_sh;
    const uint16_t* kp = a.k + b * a.k_sb + h * a.k_sh;
    const uint16_t* vp = a.v + b * a.v_sb + h * a.v_sh;
    // rows outside [0, Sq) / [0, valid) read as zeros
    const __amdgpu_buffer_rsrc_t qrs = make_rsrc(qp, (uint32_t)(a.Sq * a.q_ss * 2));
    const __amdgpu_buffer_rsrc_t krs = make_rsrc(kp, (uint32_t)(valid * a.k_ss * 2));
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(vp, (uint32_t)(valid * a.v_ss * 2));
    const __amdgpu_buffer_rsrc_t mrs =
        make_rsrc(a.kv_mask ? static_cast<const void*>(a.kv_mask + b * a.kv_mask_stride) : static_cast<const void*>(a.q),
                  a.kv_mask ? (uint32_t)((a.Sk + 3) & ~3) : 0u);

    // every load of the wave (its share, grouped) up front
    u32x4 vv[2 * KB];
#pragma unroll
    for (int j = 0; j < 2 * KB; ++j) {
        if (NW == 1 || j % NW == w) {
            const int c = lane + 64 * j;          // 16-byte chunk: key c/8, dims 8(c%8)..
            vv[j] = buffer_load16(vrs, (uint32_t)(((c >> 3) * a.v_ss + (c & 7) * 8) * 2));
        }
    }
    v8 kf[KB][2];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
        if (NW == 1 || kb % NW == w) {
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
                kf[kb][hh] = __builtin_bit_cast(
                    v8, buffer_load16(krs, (uint32_t)(((16 * kb + r) * a.k_ss + 32 * hh + 8 * g) * 2)));
        }
    }
    v8 qf[2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
        qf[hh] = __builtin_bit_cast(
            v8, buffer_load16(qrs, (uint32_t)(((q0 + r) * a.q_ss + 32 * hh + 8 * g) * 2)));
    // q_norm / k_norm weights for rows normalised as they are loaded (in the
    // kernel's element type; fp16 Q rows of a bf16 call are rounded to bf16)
    f32x4 qgm[2][2], kgm[2][2];
    load_norm_gamma(a.q_gamma, g, qgm);
    load_norm_gamma(a.k_gamma, g, kgm);
    if constexpr (!kF16) {
        if (a.q_f16) q_rows_f16_to_bf16(qf, qgm, a.q_gamma != nullptr, a.q_eps);
        else if (a.q_gamma) rms_norm_row(qf, qgm, a.q_eps);
    } else {
        if (a.q_gamma) rms_norm_row(qf, qgm, a.q_eps);
    }
    if (a.k_gamma) {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)   // the wave's blocks; those past the valid keys stay zero
            if ((NW == 1 || kb % NW == w) && 16 * kb < valid) rms_norm_row(kf[kb], kgm, a.q_eps);
    }
#pragma unroll
    for (int j = 0; j < 2 * KB; ++j) {
        if (NW == 1 || j % NW == w) {
            const int c = lane + 64 * j;
            *reinterpret_cast<u32x4*>(vl + (c >> 3) * kVPitch + (c & 7) * 8) = vv[j];
        }
    }
    if constexpr (NW > 1) {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            if (kb % NW == w) {
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) kls[(kb * 64 + lane) * 2 + hh] = __builtin_bit_cast(u32x4, kf[kb][hh]);
            }
        }
        __syncthreads();
        if (q0 >= a.Sq) return;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            if (kb % NW != w) {
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) kf[kb][hh] = __builtin_bit_cast(v8, kls[(kb * 64 + lane) * 2 + hh]);
            }
        }
    }
    asm volatile("" ::: "memory");
    // S^T blocks: lane holds keys 16kb + 4g + i of query q0 + r (raw scores)
    f32x4 s[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
        f32x4 z = {0.f, 0.f, 0.f, 0.f};
        z = mfma_in<kF16>(kf[kb][0], qf[0], z);
        s[kb] = mfma_in<kF16>(kf[kb][1], qf[1], z);
    }
    const int qrow = q0 + r;
    uint32_t mw[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) mw[kb] = a.kv_mask ? mask_word(mrs, 16 * kb + 4 * g) : 0xffffffffu;
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int key = 16 * kb + 4 * g + i;
            const bool dead = key >= valid || (a.causal && key > qrow) || ((mw[kb] >> (8 * i)) & 0xffu) == 0;
            s[kb][i] = dead ? -INFINITY : s[kb][i];
            mx = fmaxf(mx, s[kb][i]);
        }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float nm = mx == -INFINITY ? 0.f : -mx * a.scale_log2;

    // P^T as (hi, lo) pairs of the input type, O^T += V^T . P^T per 32-key step
    f32x4 acc[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    float ls = 0.f;
#pragma unroll
    for (int j = 0; j < KB / 2; ++j) {
        float pf[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            pf[t] = fast_exp2(fmaf(s[2 * j + (t >> 2)][t & 3], a.scale_log2, nm));
            ls += pf[t];
        }
        uint32_t hw[4], lw[4];
        if constexpr (kF16 || kVH) {
#pragma unroll
            for (int e = 0; e < 4; ++e) split_f16x2(pf[2 * e], pf[2 * e + 1], hw[e], lw[e]);
        } else {
            uint32_t pb[8], lb[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                pb[t] = __float_as_uint(pf[t]);
                lb[t] = __float_as_uint(pf[t] - __uint_as_float(pb[t] & 0xffff0000u));
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                hw[e] = __builtin_amdgcn_perm(pb[2 * e + 1], pb[2 * e], 0x07060302u);
                lw[e] = __builtin_amdgcn_perm(lb[2 * e + 1], lb[2 * e], 0x07060302u);
            }
        }
        // keys 32j + 4g + (0..3) and 32j + 16 + 4g + (0..3): the P^T slot order
        const uint16_t* vrow = vl + (32 * j + 4 * g + (r >> 2)) * kVPitch + 4 * (r & 3);
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            const uint2 lo4 = lds_read_tr16(vrow + 16 * db);
            const uint2 hi4 = lds_read_tr16(vrow + 16 * kVPitch + 16 * db);
            const u32x4 vw = {lo4.x, lo4.y, hi4.x, hi4.y};
            const u32x4 hv = {hw[0], hw[1], hw[2], hw[3]}, lv = {lw[0], lw[1], lw[2], lw[3]};
            if constexpr (kF16 || kVH) {
                acc[db] = mfma16x16x32_f16(u32x4_as_f16x8(vw), u32x4_as_f16x8(hv), acc[db]);
                acc[db] = mfma16x16x32_f16(u32x4_as_f16x8(vw), u32x4_as_f16x8(lv), acc[db]);
            } else {
                acc[db] = mfma16x16x32(u32x4_as_bf16x8(vw), u32x4_as_bf16x8(hv), acc[db]);
                acc[db] = mfma16x16x32(u32x4_as_bf16x8(vw), u32x4_as_bf16x8(lv), acc[db]);
            }
        }
    }
    ls += __shfl_xor(ls, 16, 64);
    ls += __shfl_xor(ls, 32, 64);
    if (qrow >= a.Sq) return;
    const float inv = ls > 0.f ? 1.f / ls : 0.f;
    // O^T lane layout: head dims 16db + 4g + i of query qrow
#pragma unroll
    for (int db = 0; db < 4; ++db)
        store_out4(a, b * a.o_sb + h * a.o_sh + qrow * a.o_ss + 16 * db + 4 * g, acc[db] * inv);
}

// ---------------------------------------------------------------------------
// fp32 Q/K/V (the reference sends fp32 to its naive kernel,
// attention.cu:90-139, 183-197): fp32 products on the fp32 MFMA
// (v_mfma_f32_16x16x4_f32), so nothing is rounded below fp32.
//
// One wave per (b, h, 16-query block, key split), K and V read straight from
// global memory (L2 serves the five query blocks of a head).  Per 16-key
// block: S^T = K.Q^T in 16 steps of 4 head dims, where step s takes dims
// 16g + s from lane group g, so each lane reads 16 contiguous dims of its
// key row and of its query row; then O^T += V^T.P^T in 4 steps, where step i
// contracts keys {4g + i}: exactly the keys whose scores the S^T accumulator
// holds in element i of lane group g, so P^T needs no shuffle, and V element
// (key 4g + i, dim 16db + r) comes from 16 consecutive floats per lane group.
// Online softmax in log2 units as in the other kernels; multi-split partials
// go to the same workspace layout and merge kernel.
// ---------------------------------------------------------------------------
__device__ __forceinline__ f32x4 mfma16x16x4_f32(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__global__ __launch_bounds__(64) void attn_f32_kernel(const AttnArgs a) {
    const int lane = threadIdx.x;
    const int g = lane >> 4;
    const int r = lane & 15;
    const int nsplit = a.nsplit;
    const int split = blockIdx.x % nsplit;
    const int q0 = 16 * (int)(blockIdx.x / nsplit);
    const int h = blockIdx.y;
    const int b = blockIdx.z;
    const int qrow = q0 + r;

    int valid = a.Sk;
    if (a.valid_len) {
        const int vl = a.valid_len[b];
        valid = vl < 0 ? 0 : (vl > a.Sk ? a.Sk : vl);
    }
    int per = (valid + nsplit - 1) / nsplit;
    per = (per + 15) & ~15;
    const int kbeg = split * per;
    int kend = min(valid, kbeg + per);
    if (a.causal) kend = min(kend, min(a.Sq, q0 + 16));

    const float* qp = reinterpret_cast<const float*>(a.q) + b * a.q_sb + h * a.q_sh;
    const float* kp = reinterpret_cast<const float*>(a.k) + b * a.k_sb + h * a.k_sh;
    const float* vp = reinterpret_cast<const float*>(a.v) + b * a.v_sb + h * a.v_sh;
    // rows outside [0, Sq) and keys outside [0, kend) read as zeros
    const __amdgpu_buffer_rsrc_t qrs = make_rsrc(qp, (uint32_t)(a.Sq * a.q_ss * 4));
    const __amdgpu_buffer_rsrc_t krs = make_rsrc(kp, (uint32_t)(max(kend, 0) * a.k_ss * 4));
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(vp, (uint32_t)(max(kend, 0) * a.v_ss * 4));
    const __amdgpu_buffer_rsrc_t mrs =
        make_rsrc(a.kv_mask ? static_cast<const void*>(a.kv_mask + b * a.kv_mask_stride) : static_cast<const void*>(a.q),
                  a.kv_mask ? (uint32_t)((a.Sk + 3) & ~3) : 0u);

    float qv[16];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const u32x4 w = buffer_load16(qrs, (uint32_t)((qrow * a.q_ss + 16 * g + 4 * c) * 4));
#pragma unroll
        for (int e = 0; e < 4; ++e) qv[4 * c + e] = __uint_as_float(w[e]);
    }
    f32x4 acc[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY;   // running row max, log2 units
    float l = 0.f;         // this lane's share of the row sum
    for (int kt = kbeg; kt < kend; kt += 16) {
        float kv[16], vv[16];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const u32x4 w = buffer_load16(krs, (uint32_t)(((kt + r) * a.k_ss + 16 * g + 4 * c) * 4));
#pragma unroll
            for (int e = 0; e < 4; ++e) kv[4 * c + e] = __uint_as_float(w[e]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int db = 0; db < 4; ++db)
                vv[4 * i + db] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                    vrs, (uint32_t)(((kt + 4 * g + i) * a.v_ss + 16 * db + r) * 4), 0, 0));
        const uint32_t mw = a.kv_mask ? mask_word(mrs, kt + 4 * g) : 0xffffffffu;
        f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < 16; ++st) sc = mfma16x16x4_f32(kv[st], qv[st], sc);
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int key = kt + 4 * g + i;
            const bool dead = key >= kend || (a.causal && key > qrow) || ((mw >> (8 * i)) & 0xffu) == 0;
            sc[i] = dead ? -INFINITY : sc[i] * a.scale_log2;
            mx = fmaxf(mx, sc[i]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mnew = fmaxf(m, mx);
        const float muse = mnew == -INFINITY ? 0.f : mnew;
        const float alpha = fast_exp2(m - muse);
        m = mnew;
        l *= alpha;
#pragma unroll
        for (int db = 0; db < 4; ++db) acc[db] *= alpha;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float p = fast_exp2(sc[i] - muse);
            l += p;
#pragma unroll
            for (int db = 0; db < 4; ++db) acc[db] = mfma16x16x4_f32(vv[4 * i + db], p, acc[db]);
        }
    }
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    if (qrow >= a.Sq) return;
    // O^T lane layout: head dims 16db + 4g + i of query qrow
    if (nsplit == 1) {
        const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
        for (int db = 0; db < 4; ++db)
            store_out4(a, b * a.o_sb + h * a.o_sh + qrow * a.o_ss + 16 * db + 4 * g, acc[db] * inv);
    } else {
        const size_t row = (((size_t)b * a.H + h) * nsplit + split) * (size_t)a.Sq + qrow;
#pragma unroll
        for (int db = 0; db < 4; ++db)
            *reinterpret_cast<f32x4*>(a.part_o + row * kD + 16 * db + 4 * g) = acc[db];
        if (g == 0) *reinterpret_cast<float2*>(a.part_ml + row * 2) = float2{m, l};
    }
}

}  // namespace sfk

// ---------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------
namespace {

using sfk::kMaxSplits;

int query_chunks(const sf_attn_desc* d) { return (d->Sq + 16 * sfk::kQB - 1) / (16 * sfk::kQB); }

// Keys up to which a grid that leaves CUs idle runs one workgroup per 16-row
// query block (all of a head's keys each, no split, no merge pass) instead
// of key splits.
constexpr int kQGroupMaxKeys = 1024;

// MI355X has 256 CUs.  When B*H*query-chunks alone fills them the keys are
// not split (no partials, no merge pass: measured faster at B = 8 and 16 than
// two splits).  Otherwise the keys are split so that the grid is about one
// workgroup per CU, and then into the fewest splits whose longest split has
// the same number of 128-key tiles (image keys at B = 1: 35 tiles, 8 splits
// of <= 5 tiles -> 7 splits).  Measured at B = 1 on 4374 keys: 7 splits
// 20.3 us, 8 21.0, 12 22.1, 16 (two workgroups per CU) 24.8; at B = 2, 4
// splits 26.5 us against 29.3 for 8: a workgroup alone on its CU contracts
// its tiles at the CU's full rate, and fewer splits halve the partials the
// merge pass reads.  At B = 1 on 1024 keys (8 tiles), 4 splits of 2 tiles
// took 10.1 us against 10.8 for 8 of one tile.
constexpr long kNumCUs = 256;

int choose_splits(const sf_attn_desc* d) {
    if (d->num_splits > 0) return d->num_splits < kMaxSplits ? d->num_splits : kMaxSplits;
    const long base = (long)d->B * d->H * query_chunks(d);
    if (base <= 0) return 1;
    if (base >= kNumCUs) return 1;
    if (d->Sk <= kQGroupMaxKeys && d->in_dtype != SF_F32) return 1;   // query blocks instead
    const long tiles = ((long)d->Sk + 127) / 128;
    long ns = kNumCUs / base;
    // at least two tiles per split: one-tile splits cost their fixed start
    // and epilogue for one tile's work and double the partials to merge
    if (ns > (tiles + 1) / 2) ns = (tiles + 1) / 2;
    if (ns < 1) ns = 1;
    const long longest = (tiles + ns - 1) / ns;
    ns = (tiles + longest - 1) / longest;
    if (ns > kMaxSplits) ns = kMaxSplits;
    return (int)ns;
}

template <int NW, bool F16, bool VH>
void launch_short_kb(int kb, dim3 grid, hipStream_t s, const sfk::AttnArgs& a) {
    const dim3 block(64 * NW);
    if (kb <= 2) hipLaunchKernelGGL((sfk::attn_short_kernel<2, F16, NW, VH>), grid, block, 0, s, a);
    else if (kb <= 4) hipLaunchKernelGGL((sfk::attn_short_kernel<4, F16, NW, VH>), grid, block, 0, s, a);
    else if (kb <= 6) hipLaunchKernelGGL((sfk::attn_short_kernel<6, F16, NW, VH>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((sfk::attn_short_kernel<8, F16, NW, VH>), grid, block, 0, s, a);
}

// vh: bf16 Q/K with fp16 V (sf_attn_desc.v_f16)
template <int NW>
void launch_short(bool f16, bool vh, int kb, dim3 grid, hipStream_t s, const sfk::AttnArgs& a) {
    if (f16) launch_short_kb<NW, true, false>(kb, grid, s, a);
    else if (vh) launch_short_kb<NW, false, true>(kb, grid, s, a);
    else launch_short_kb<NW, false, false>(kb, grid, s, a);
}

// QB: 16-row query blocks per workgroup (kQB: 80-row chunks on a (split x
// chunk, H, B) grid; 1: the XCD-grouped 1-D query-block grid).
// vh: bf16 Q/K with fp16 V (sf_attn_desc.v_f16; fp16 P.V form only).
template <int QB>
void launch_ring(bool exact, bool f16, bool vh, dim3 grid, hipStream_t s, const sfk::AttnArgs& a) {
    if (exact) {
        if (f16) hipLaunchKernelGGL((sfk::attn_ring_kernel<true, true, QB>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((sfk::attn_ring_kernel<true, false, QB>), grid, dim3(256), 0, s, a);
    } else if (vh) {
        hipLaunchKernelGGL((sfk::attn_ring_kernel<false, false, QB, false, true>), grid, dim3(256), 0, s, a);
    } else {
        if (f16) hipLaunchKernelGGL((sfk::attn_ring_kernel<false, true, QB>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((sfk::attn_ring_kernel<false, false, QB>), grid, dim3(256), 0, s, a);
    }
}

// The query-block grid with Q finished from split-K partials (bf16).
void launch_ring_qp(bool exact, bool vh, dim3 grid, hipStream_t s, const sfk::AttnArgs& a) {
    if (exact) hipLaunchKernelGGL((sfk::attn_ring_kernel<true, false, 1, true>), grid, dim3(256), 0, s, a);
    else if (vh) hipLaunchKernelGGL((sfk::attn_ring_kernel<false, false, 1, true, true>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((sfk::attn_ring_kernel<false, false, 1, true>), grid, dim3(256), 0, s, a);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int validate(const sf_attn_desc* d) {
    if (!d) return SF_EINVAL;
    if (d->B < 0 || d->H < 0 || d->Sq < 0 || d->Sk < 0) return SF_EINVAL;
    if (d->D != sfk::kD) return SF_ENOTSUP;
    if (d->in_dtype != SF_BF16 && d->in_dtype != SF_F16 && d->in_dtype != SF_F32) return SF_ENOTSUP;
    if (d->out_dtype != SF_BF16 && d->out_dtype != SF_F32 && d->out_dtype != SF_F16) return SF_ENOTSUP;
    if (d->num_splits < 0) return SF_EINVAL;
    if (!(d->scale >= 0.f)) return SF_ENOTSUP;   // negative or NaN scale
    // Every stride a non-negative multiple of 8 elements (16-byte rows for
    // the vector loads and stores); rows along s at least D apart (the
    // kernels address a head's rows through one buffer range of S * s-stride).
    const int64_t* st[4] = {d->q_stride, d->k_stride, d->v_stride, d->o_stride};
    for (int i = 0; i < 4; ++i) {
        for (int j = 0; j < 3; ++j)
            if (st[i][j] < 0 || (st[i][j] & 7)) return SF_EINVAL;
        if (st[i][2] < d->D) return SF_EINVAL;
    }
    if (d->Sk == 0 && d->B > 0 && d->H > 0 && d->Sq > 0) return SF_EINVAL;
    if (d->kv_mask && ((reinterpret_cast<uintptr_t>(d->kv_mask) & 3) || (d->kv_mask_stride & 3) ||
                       (d->B > 1 && d->kv_mask_stride < d->Sk)))
        return SF_EINVAL;
    if (d->q_partials) {   // Q finished from its projection's split-K partials
        if (d->in_dtype != SF_BF16) return SF_ENOTSUP;
        if (d->q_splits < 1 || d->q_splits > 8) return SF_EINVAL;
        const void* ptrs[4] = {d->q_partials, d->q_bias, d->q_scale, d->q_gamma};
        for (const void* p : ptrs)
            if (reinterpret_cast<uintptr_t>(p) & 15) return SF_EINVAL;
        if ((int64_t)d->q_splits * d->B * d->Sq * d->H * 64 * 4 > 0x7fffffffLL) return SF_ENOTSUP;
        if (d->q_row_ss && (d->q_row_tiles < 1 || d->q_row_tiles > 64 || d->q_row_n <= 0 || !(d->q_row_eps >= 0.f)))
            return SF_EINVAL;
    } else if (d->q_row_ss) {
        return SF_EINVAL;   // a row scale applies to Q given as partials only
    }
    if (d->q_f16) {   // fp16 Q rows against bf16 K / V
        if (d->in_dtype != SF_BF16 || d->q_partials) return SF_ENOTSUP;
    }
    if (d->v_f16) {   // fp16 V against bf16 Q / K, fp16 P.V form
        if (d->in_dtype != SF_BF16 || d->exact_pv) return SF_ENOTSUP;
    }
    if (d->q_gamma || d->k_gamma) {   // per-head Q / K RMSNorm on load
        if (d->in_dtype == SF_F32) return SF_ENOTSUP;
        if ((reinterpret_cast<uintptr_t>(d->q_gamma) & 15) || (reinterpret_cast<uintptr_t>(d->k_gamma) & 15))
            return SF_EINVAL;
        // K rows are normalised by the short-key kernel only (the key-split
        // kernels stream K tiles straight into LDS)
        const bool short_keys = d->Sk <= sfk::kShortMaxKeys && d->num_splits <= 1 && !d->q_partials;
        if (d->k_gamma && !short_keys) return SF_ENOTSUP;
    }
    // Per-head byte ranges are addressed with 32-bit buffer offsets.
    const int64_t es = d->in_dtype == SF_F32 ? 4 : 2;
    if ((int64_t)d->Sq * d->q_stride[2] * es > 0x7fffffffLL ||
        (int64_t)d->Sk * d->k_stride[2] * es > 0x7fffffffLL ||
        (int64_t)d->Sk * d->v_stride[2] * es > 0x7fffffffLL)
        return SF_ENOTSUP;
    return SF_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// Allocation-free variant: the split-K partials live in a fixed device array
// instead of a caller workspace.  Every auto-chosen split count keeps the
// partials under ~5.4 MB (B*H*chunks*splits is about one workgroup per CU,
// 256 x 80 rows x 66 floats), so only a forced num_splits can exceed it.
// ---------------------------------------------------------------------------
static __device__ __align__(256) char scratch[SF_ATTN_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};   // device address of `scratch`, per device

// The device address of this device's copy of `scratch`, looked up once per
// device (with that device current) on its first use.  Host code never
// passes the array's name itself to a kernel: on the host that name is a
// stand-in, not a device address.
int scratch_address(void** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return SF_EDEVICE;
    if (dev < 0 || dev >= kMaxDevices) return SF_ENOTSUP;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return SF_EDEVICE;
        g_scratch_dev[dev] = p;
    }
    *out = g_scratch_dev[dev];
    return SF_OK;
}

}  // namespace

extern "C" int sf_attn_fwd_noalloc(const sf_attn_desc* d, const void* q, const void* k, const void* v,
                                   void* out, void* stream) {
    const int st = validate(d);
    if (st != SF_OK) return st;
    const size_t need = sf_attn_workspace_bytes(d);
    if (need > (size_t)SF_ATTN_NOALLOC_SCRATCH_BYTES) return SF_ESCRATCH;
    void* ws = nullptr;
    if (need > 0) {
        const int sst = scratch_address(&ws);
        if (sst != SF_OK) return sst;
    }
    return sf_attn_fwd(d, q, k, v, out, ws, need, stream);
}

extern "C" void sf_attn_desc_init_bhsd(sf_attn_desc* d, int32_t B, int32_t H, int32_t Sq,
                                       int32_t Sk, int32_t D, int32_t in_dtype,
                                       int32_t out_dtype) {
    if (!d) return;
    *d = sf_attn_desc{};
    d->B = B; d->H = H; d->Sq = Sq; d->Sk = Sk; d->D = D;
    d->scale = 0.f;
    d->in_dtype = in_dtype;
    d->out_dtype = out_dtype;
    d->q_stride[0] = (int64_t)H * Sq * D; d->q_stride[1] = (int64_t)Sq * D; d->q_stride[2] = D;
    d->k_stride[0] = (int64_t)H * Sk * D; d->k_stride[1] = (int64_t)Sk * D; d->k_stride[2] = D;
    d->v_stride[0] = d->k_stride[0]; d->v_stride[1] = d->k_stride[1]; d->v_stride[2] = D;
    d->o_stride[0] = d->q_stride[0]; d->o_stride[1] = d->q_stride[1]; d->o_stride[2] = D;
}

extern "C" int32_t sf_attn_num_splits(const sf_attn_desc* d) {
    if (validate(d) != SF_OK) return 0;
    if (d->Sk <= sfk::kShortMaxKeys && d->num_splits <= 1) return 1;
    return choose_splits(d);
}

extern "C" size_t sf_attn_workspace_bytes(const sf_attn_desc* d) {
    if (validate(d) != SF_OK) return 0;
    if (d->Sk <= sfk::kShortMaxKeys && d->num_splits <= 1) return 0;
    const int ns = choose_splits(d);
    if (ns <= 1) return 0;
    const size_t rows = (size_t)d->B * d->H * ns * d->Sq;
    return rows * (sfk::kD + 2) * sizeof(float);
}

extern "C" int sf_attn_fwd(const sf_attn_desc* d, const void* q, const void* k, const void* v,
                           void* out, void* workspace, size_t workspace_bytes, void* stream) {
    int st = validate(d);
    if (st != SF_OK) return st;
    if ((long)d->B * d->H * d->Sq == 0) return SF_OK;
    const bool q_from_partials = d->q_partials != nullptr;
    if (!q_from_partials && !q) return SF_EINVAL;
    if (!k || !v || !out) return SF_EINVAL;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out)) return SF_EINVAL;
    if (d->B > 65535 || d->H > 65535) return SF_ENOTSUP;

    // (Q from partials runs the query-block grid whatever the key count)
    const bool short_keys = d->Sk <= sfk::kShortMaxKeys && d->num_splits <= 1 && !q_from_partials;
    const int ns = short_keys ? 1 : choose_splits(d);
    // one workgroup per 16-row query block: no key split, and a grid of
    // 80-row chunks that would leave CUs idle
    const long bh = (long)d->B * d->H;
    const bool qblocks = !short_keys && ns == 1 && d->in_dtype != SF_F32 && d->Sk <= kQGroupMaxKeys &&
                         bh * query_chunks(d) < kNumCUs;
    const int nqc = qblocks ? (d->Sq + 15) / 16 : query_chunks(d);
    if (q_from_partials && !qblocks) return SF_ENOTSUP;
    sfk::AttnArgs a{};
    a.q = static_cast<const uint16_t*>(q_from_partials && !q ? k : q);   // not read with partials
    if (q_from_partials) {
        a.qp = d->q_partials;
        a.q_splits = d->q_splits;
        a.qp_bytes = (uint32_t)((int64_t)d->q_splits * d->B * d->Sq * d->H * 64 * 4);
        a.q_bias = d->q_bias;
        a.q_scale = d->q_scale;
    }
    a.q_gamma = d->q_gamma;
    a.q_eps = d->q_eps;
    a.k_gamma = d->k_gamma;
    a.q_f16 = d->q_f16 != 0;
    a.q_row_ss = d->q_row_ss;
    a.q_row_tiles = d->q_row_tiles;
    a.q_row_inv_n = d->q_row_n > 0 ? 1.f / (float)d->q_row_n : 0.f;
    a.q_row_eps = d->q_row_eps;
    a.k = static_cast<const uint16_t*>(k);
    a.v = static_cast<const uint16_t*>(v);
    a.o = out;
    a.valid_len = d->kv_valid_len;
    a.kv_mask = d->kv_mask;
    a.kv_mask_stride = d->kv_mask_stride;
    a.q_sb = d->q_stride[0]; a.q_sh = d->q_stride[1]; a.q_ss = d->q_stride[2];
    a.k_sb = d->k_stride[0]; a.k_sh = d->k_stride[1]; a.k_ss = d->k_stride[2];
    a.v_sb = d->v_stride[0]; a.v_sh = d->v_stride[1]; a.v_ss = d->v_stride[2];
    a.o_sb = d->o_stride[0]; a.o_sh = d->o_stride[1]; a.o_ss = d->o_stride[2];
    a.B = d->B; a.H = d->H; a.Sq = d->Sq; a.Sk = d->Sk;
    a.nsplit = ns;
    a.nqc = nqc;
    a.out_kind = d->out_dtype == SF_F32 ? sfk::kOutF32 : (d->out_dtype == SF_F16 ? sfk::kOutF16 : sfk::kOutBF16);
    a.causal = d->is_causal != 0;
    const float scale = d->scale != 0.f ? d->scale : 1.f / sqrtf((float)d->D);
    a.scale_log2 = scale * 1.4426950408889634f;
    if (ns > 1) {
        const size_t need = sf_attn_workspace_bytes(d);
        if (!workspace || workspace_bytes < need || !aligned16(workspace)) return SF_EWORKSPACE;
        a.part_o = static_cast<float*>(workspace);
        a.part_ml = a.part_o + (size_t)d->B * d->H * ns * d->Sq * sfk::kD;
    }
    if ((long)ns * nqc > 0x7fffffffL) return SF_ENOTSUP;

    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool f16 = d->in_dtype == SF_F16;
    const bool vh = d->v_f16 != 0;
    if (d->in_dtype == SF_F32) {
        const long qblocks = (d->Sq + 15) / 16;
        if ((long)ns * qblocks > 0x7fffffffL) return SF_ENOTSUP;
        hipLaunchKernelGGL(sfk::attn_f32_kernel, dim3((unsigned)(ns * qblocks), d->H, d->B), dim3(64), 0, s, a);
    } else if (short_keys) {
        const int qb = (d->Sq + 15) / 16;
        const int kb = ((d->Sk + 31) / 32) * 2;
        // one wave per query block while B*H < 256 leaves CUs idle; from
        // B*H >= 256 (every batch size) a head's query blocks are the five
        // waves of one workgroup sharing K and V in LDS
        const long bh = (long)d->B * d->H;
        const bool grouped = bh >= sfk::kShortGroupMinHeads;
        if (grouped)
            launch_short<5>(f16, vh, kb, dim3((qb + 4) / 5, d->H, d->B), s, a);
        else
            launch_short<1>(f16, vh, kb, dim3(qb, d->H, d->B), s, a);
        return hipGetLastError() == hipSuccess ? SF_OK : SF_ELAUNCH;
    } else {
        if (qblocks) {
            const long groups = (bh + 7) / 8;
            if (8L * nqc * groups > 0x7fffffffL) return SF_ENOTSUP;
            const dim3 grid((unsigned)(8L * nqc * groups));
            if (q_from_partials) launch_ring_qp(d->exact_pv != 0, vh, grid, s, a);
            else launch_ring<1>(d->exact_pv != 0, f16, vh, grid, s, a);
        } else {
            launch_ring<sfk::kQB>(d->exact_pv != 0, f16, vh, dim3(ns * nqc, d->H, d->B), s, a);
        }
    }
    if (hipGetLastError() != hipSuccess) return SF_ELAUNCH;
    if (ns > 1) {
        hipLaunchKernelGGL(sfk::attn_merge_kernel, dim3((d->Sq + 3) / 4, d->H, d->B), dim3(256), 0,
                           s, a);
        if (hipGetLastError() != hipSuccess) return SF_ELAUNCH;
    }
    return SF_OK;
}

extern "C" const char* sf_strerror(int status) {
    switch (status) {
        case SF_OK: return "success";
        case SF_EINVAL: return "invalid argument (shape, stride, alignment or pointer)";
        case SF_ENOTSUP: return "unsupported configuration (dtype, head dim or size)";
        case SF_EWORKSPACE: return "workspace missing or too small";
        case SF_ELAUNCH: return "kernel launch failed";
        case SF_EDEVICE: return "HIP runtime error";
        case SF_ESCRATCH: return "request exceeds the fixed device scratch of the allocation-free entry point";
        default: return "unknown status";
    }
}
