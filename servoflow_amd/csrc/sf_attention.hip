// Attention for the RDT-1B denoise loop on MI355X (gfx950).
//
// Replaces the attention op behind IBackend::attention
// (include/servoflow/backend/backend.h:105-110): CUDABackend::attention
// (src/backend/cuda/cuda_backend.cu:470-501) -> cuda_ops::flash_attention
// (src/backend/cuda/ops/attention.cu:183-197), whose arithmetic is the
// online-softmax loop of naive_attention_kernel (attention.cu:90-139).
//
// Design (one kernel family serves the 67x67 self-attention and the
// 67 x 4374 / 67 x <=1024 cross-attention):
//   * grid = (splits x query-chunks, H, B); a workgroup of 4 waves owns one
//     (b, h, query chunk of 80 rows, key split).  Splitting the keys
//     (flash-decoding) is what fills 256 CUs when B*H = 32.
//   * K/V tiles of 128 keys are streamed HBM -> VGPR -> LDS with 16-byte
//     coalesced loads, double-buffered so the next tile's loads are in
//     flight while the current tile is contracted.
//   * Each wave contracts 32 keys of the tile against all 80 query rows with
//     v_mfma_f32_16x16x32_bf16: S^T = K.Q^T, then O^T += V^T.P^T.  The S^T
//     accumulator layout (lane = query, 4 consecutive keys per lane) is
//     directly the B operand P^T, so no shuffle sits between the two
//     contractions.
//   * P is carried as a bf16 (hi, lo) pair so the P.V contraction keeps ~16
//     mantissa bits; a single bf16 P costs ~1.1e-3 mean relative error on
//     its own, which is the whole 1e-3 budget.
//   * Online softmax in the log2 domain; the four waves' (m, l, O) merge in
//     LDS; multi-split partials merge in a second small kernel.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "sf_device.h"
#include "sf_hip.h"

namespace sfk {

constexpr int kKT = 128;    // keys per tile per workgroup (4 waves x 32)
constexpr int kRow = 72;    // LDS row pitch in bf16 elements (144 B, bank-skewed)
constexpr int kD = 64;      // head dim this kernel family is built for
constexpr int kQB = 5;      // 16-row query blocks per workgroup (80 rows >= 67)
constexpr int kThreads = 256;

struct AttnArgs {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    void* o;
    float* part_o;    // [B*H][nsplit][Sq][64] unnormalised outputs
    float* part_ml;   // [B*H][nsplit][Sq][2]  (running max in log2 units, sum)
    const int32_t* valid_len;
    int64_t q_sb, q_sh, q_ss;
    int64_t k_sb, k_sh, k_ss;
    int64_t v_sb, v_sh, v_ss;
    int64_t o_sb, o_sh, o_ss;
    int B, H, Sq, Sk;
    int nsplit;
    int out_f32;
    int causal;
    float scale_log2;   // scale * log2(e)
};

__device__ __forceinline__ void store_out(const AttnArgs& a, int b, int h, int q,
                                          int d, float val) {
    const int64_t off = b * a.o_sb + h * a.o_sh + q * a.o_ss + d;
    if (a.out_f32) {
        reinterpret_cast<float*>(a.o)[off] = val;
    } else {
        reinterpret_cast<uint16_t*>(a.o)[off] = (uint16_t)f32_to_bf16_bits(val);
    }
}

// One (b, h, query chunk, key split) per workgroup.
__global__ __launch_bounds__(kThreads) void attn_split_kernel(const AttnArgs a) {
    constexpr int QR = 16 * kQB;
    constexpr int kTileElems = kKT * kRow;
    __shared__ __attribute__((aligned(16))) uint16_t lds[2 * 2 * kTileElems];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int g = lane >> 4;
    const int r = lane & 15;
    const int nsplit = a.nsplit;
    const int split = blockIdx.x % nsplit;
    const int qc = blockIdx.x / nsplit;
    const int h = blockIdx.y;
    const int b = blockIdx.z;
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

    // Q as the B operand of S^T = K.Q^T: lane holds query row (16qb + r),
    // head-dim elements [32dc + 8g, +8).
    bf16x8 qf[kQB][2];
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
        const int row = q0 + 16 * qb + r;
#pragma unroll
        for (int dc = 0; dc < 2; ++dc) {
            qf[qb][dc] = row < a.Sq ? load_bf16x8(qp + row * a.q_ss + 32 * dc + 8 * g)
                                    : zero_bf16x8();
        }
    }

    f32x4 acc[kQB][4];   // O^T blocks: lane holds d = 16db + 4g + i, q = 16qb + r
    float m[kQB], l[kQB];
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
        m[qb] = -INFINITY;
        l[qb] = 0.f;
#pragma unroll
        for (int db = 0; db < 4; ++db) acc[qb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // Global -> register prefetch of one tile: 1024 16-byte chunks of K and
    // of V, four of each per thread; 8 threads cover one 128-byte key row.
    u32x4 pk[4], pv[4];
    auto gload = [&](int kt) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = tid + kThreads * j;
            const int row = c >> 3;
            const int col = (c & 7) * 8;
            const int key = kt + row;
            if (key < kend) {
                pk[j] = *reinterpret_cast<const u32x4*>(kp + key * a.k_ss + col);
                pv[j] = *reinterpret_cast<const u32x4*>(vp + key * a.v_ss + col);
            } else {
                pk[j] = u32x4{0u, 0u, 0u, 0u};
                pv[j] = u32x4{0u, 0u, 0u, 0u};
            }
        }
    };
    auto lstore = [&](int buf) {
        uint16_t* kl = lds + buf * 2 * kTileElems;
        uint16_t* vl = kl + kTileElems;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = tid + kThreads * j;
            const int row = c >> 3;
            const int col = (c & 7) * 8;
            *reinterpret_cast<u32x4*>(kl + row * kRow + col) = pk[j];
            *reinterpret_cast<u32x4*>(vl + row * kRow + col) = pv[j];
        }
    };

    if (ntiles > 0) {
        gload(kbeg);
        lstore(0);
    }
    __syncthreads();

    for (int t = 0; t < ntiles; ++t) {
        const int kt = kbeg + t * kKT;
        if (t + 1 < ntiles) gload(kt + kKT);

        const uint16_t* kl = lds + (t & 1) * 2 * kTileElems;
        const uint16_t* vl = kl + kTileElems;
        const int wkey = 32 * w;   // this wave's first key inside the tile

        // ---- S^T = K . Q^T for the wave's 32 keys (two 16-key blocks).
        f32x4 s[2][kQB];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const uint16_t* krow = kl + (wkey + 16 * kb + r) * kRow + 8 * g;
            const bf16x8 k0 = load_bf16x8(krow);
            const bf16x8 k1 = load_bf16x8(krow + 32);
#pragma unroll
            for (int qb = 0; qb < kQB; ++qb) {
                f32x4 z = {0.f, 0.f, 0.f, 0.f};
                z = mfma16x16x32(k0, qf[qb][0], z);
                s[kb][qb] = mfma16x16x32(k1, qf[qb][1], z);
            }
        }

        // ---- V^T fragments: lane holds d = 16db + r and the 8 keys
        //      {4g..4g+3, 16+4g..16+4g+3} of the wave's 32 (the same key
        //      order the S^T accumulator gives P^T).
        bf16x8 vf[4];
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            uint16_t e[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int key = wkey + (j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4));
                e[j] = vl[key * kRow + 16 * db + r];
            }
            u32x4 pw;
            pw.x = (uint32_t)e[0] | ((uint32_t)e[1] << 16);
            pw.y = (uint32_t)e[2] | ((uint32_t)e[3] << 16);
            pw.z = (uint32_t)e[4] | ((uint32_t)e[5] << 16);
            pw.w = (uint32_t)e[6] | ((uint32_t)e[7] << 16);
            vf[db] = u32x4_as_bf16x8(pw);
        }

        const bool need_mask = a.causal || (kt + kKT > kend);
#pragma unroll
        for (int qb = 0; qb < kQB; ++qb) {
            const int qrow = q0 + 16 * qb + r;
            float x[8];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float v = s[kb][qb][i] * a.scale_log2;
                    if (need_mask) {
                        const int key = kt + wkey + 16 * kb + 4 * g + i;
                        const bool dead = key >= kend || (a.causal && key > qrow);
                        v = dead ? -INFINITY : v;
                    }
                    x[4 * kb + i] = v;
                }
            }
            float mx = x[0];
#pragma unroll
            for (int j = 1; j < 8; ++j) mx = fmaxf(mx, x[j]);
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float mnew = fmaxf(m[qb], mx);
            const float muse = mnew == -INFINITY ? 0.f : mnew;
            const float alpha = fast_exp2(m[qb] - muse);
            m[qb] = mnew;
            float ls = l[qb] * alpha;
#pragma unroll
            for (int db = 0; db < 4; ++db) acc[qb][db] *= alpha;

            // P = exp2(x - m) split into bf16 hi (truncated) + bf16 lo.
            uint32_t hi[8], lo[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float p = fast_exp2(x[j] - muse);
                ls += p;
                const uint32_t pb = __float_as_uint(p);
                const uint32_t ph = pb & 0xffff0000u;
                hi[j] = ph;
                lo[j] = __float_as_uint(p - __uint_as_float(ph)) & 0xffff0000u;
            }
            l[qb] = ls;
            u32x4 phw, plw;
            phw.x = (hi[0] >> 16) | hi[1];
            phw.y = (hi[2] >> 16) | hi[3];
            phw.z = (hi[4] >> 16) | hi[5];
            phw.w = (hi[6] >> 16) | hi[7];
            plw.x = (lo[0] >> 16) | lo[1];
            plw.y = (lo[2] >> 16) | lo[3];
            plw.z = (lo[4] >> 16) | lo[5];
            plw.w = (lo[6] >> 16) | lo[7];
            const bf16x8 ph8 = u32x4_as_bf16x8(phw);
            const bf16x8 pl8 = u32x4_as_bf16x8(plw);
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                acc[qb][db] = mfma16x16x32(vf[db], ph8, acc[qb][db]);
                acc[qb][db] = mfma16x16x32(vf[db], pl8, acc[qb][db]);
            }
        }

        if (t + 1 < ntiles) lstore((t + 1) & 1);
        __syncthreads();
    }

    // ---- Row sums: each lane summed its own 8 keys per tile; add the four
    //      lane groups that share a query.
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
        l[qb] += __shfl_xor(l[qb], 16, 64);
        l[qb] += __shfl_xor(l[qb], 32, 64);
    }

    // ---- Merge the four waves' (m, l, O) through LDS (tile buffers reused).
    float* sm = reinterpret_cast<float*>(lds);   // [4][QR]
    float* sl = sm + 4 * QR;                     // [4][QR]
    float* sM = sl + 4 * QR;                     // [QR] merged max
    float* sL = sM + QR;                         // [QR] merged sum
    float* so = sL + QR;                         // [4][QR][32] half of O
    if (g == 0) {
#pragma unroll
        for (int qb = 0; qb < kQB; ++qb) {
            sm[w * QR + 16 * qb + r] = m[qb];
            sl[w * QR + 16 * qb + r] = l[qb];
        }
    }
    __syncthreads();
    if (tid < QR) {
        float M = sm[tid];
        for (int ww = 1; ww < 4; ++ww) M = fmaxf(M, sm[ww * QR + tid]);
        const float Muse = M == -INFINITY ? 0.f : M;
        float L = 0.f;
        for (int ww = 0; ww < 4; ++ww) L += sl[ww * QR + tid] * fast_exp2(sm[ww * QR + tid] - Muse);
        sM[tid] = M;
        sL[tid] = L;
    }
    __syncthreads();
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
        const float M = sM[16 * qb + r];
        const float Muse = M == -INFINITY ? 0.f : M;
        const float f = fast_exp2(m[qb] - Muse);
#pragma unroll
        for (int db = 0; db < 4; ++db) acc[qb][db] *= f;
    }

    const size_t bh = (size_t)b * a.H + h;
    const size_t pbase = (bh * nsplit + split) * (size_t)a.Sq;
    for (int half = 0; half < 2; ++half) {
#pragma unroll
        for (int qb = 0; qb < kQB; ++qb) {
#pragma unroll
            for (int dbh = 0; dbh < 2; ++dbh) {
                const int db = 2 * half + dbh;
                float* dst = so + (w * QR + 16 * qb + r) * 32 + 16 * dbh + 4 * g;
                *reinterpret_cast<f32x4*>(dst) = acc[qb][db];
            }
        }
        __syncthreads();
        for (int idx = tid; idx < QR * 32; idx += kThreads) {
            const int qq = idx >> 5;
            const int dd = idx & 31;
            const int qrow = q0 + qq;
            if (qrow < a.Sq) {
                float val = so[qq * 32 + dd] + so[(QR + qq) * 32 + dd] +
                            so[(2 * QR + qq) * 32 + dd] + so[(3 * QR + qq) * 32 + dd];
                const int d = 32 * half + dd;
                if (nsplit == 1) {
                    const float L = sL[qq];
                    store_out(a, b, h, qrow, d, L > 0.f ? val / L : 0.f);
                } else {
                    a.part_o[(pbase + qrow) * kD + d] = val;
                }
            }
        }
        __syncthreads();
    }
    if (nsplit > 1 && tid < QR && q0 + tid < a.Sq) {
        a.part_ml[(pbase + q0 + tid) * 2 + 0] = sM[tid];
        a.part_ml[(pbase + q0 + tid) * 2 + 1] = sL[tid];
    }
}

// Log-sum-exp merge of the split partials: one thread per (q, d).
__global__ __launch_bounds__(256) void attn_merge_kernel(const AttnArgs a) {
    const int tid = threadIdx.x;
    const int q = blockIdx.x * 4 + (tid >> 6);
    const int d = tid & 63;
    const int h = blockIdx.y;
    const int b = blockIdx.z;
    if (q >= a.Sq) return;
    const int ns = a.nsplit;
    const size_t bh = (size_t)b * a.H + h;
    float M = -INFINITY;
    for (int s = 0; s < ns; ++s)
        M = fmaxf(M, a.part_ml[((bh * ns + s) * a.Sq + q) * 2]);
    const float Muse = M == -INFINITY ? 0.f : M;
    float L = 0.f, O = 0.f;
    for (int s = 0; s < ns; ++s) {
        const size_t row = (bh * ns + s) * a.Sq + q;
        const float f = fast_exp2(a.part_ml[row * 2] - Muse);
        L += f * a.part_ml[row * 2 + 1];
        O += f * a.part_o[row * kD + d];
    }
    store_out(a, b, h, q, d, L > 0.f ? O / L : 0.f);
}

}  // namespace sfk

// ---------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------
namespace {

constexpr int kMaxSplits = 64;

int query_chunks(const sf_attn_desc* d) { return (d->Sq + 16 * sfk::kQB - 1) / (16 * sfk::kQB); }

int choose_splits(const sf_attn_desc* d) {
    if (d->num_splits > 0) return d->num_splits < kMaxSplits ? d->num_splits : kMaxSplits;
    const long base = (long)d->B * d->H * query_chunks(d);
    if (base <= 0) return 1;
    // Aim for ~2 workgroups per CU on a 256-CU part, with >= 256 keys a split.
    long want = (512 + base - 1) / base;
    long cap = d->Sk / 256;
    long ns = want < cap ? want : cap;
    if (ns < 1) ns = 1;
    if (ns > kMaxSplits) ns = kMaxSplits;
    return (int)ns;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int validate(const sf_attn_desc* d) {
    if (!d) return SF_EINVAL;
    if (d->B < 0 || d->H < 0 || d->Sq < 0 || d->Sk < 0) return SF_EINVAL;
    if (d->D != sfk::kD) return SF_ENOTSUP;
    if (d->in_dtype != SF_BF16) return SF_ENOTSUP;
    if (d->out_dtype != SF_BF16 && d->out_dtype != SF_F32) return SF_ENOTSUP;
    if (d->num_splits < 0) return SF_EINVAL;
    const int64_t* st[4] = {d->q_stride, d->k_stride, d->v_stride, d->o_stride};
    for (int i = 0; i < 3; ++i)
        for (int j = 0; j < 3; ++j)
            if (st[i][j] < 0 || (st[i][j] & 7)) return SF_EINVAL;
    for (int j = 0; j < 3; ++j)
        if (d->o_stride[j] < 0) return SF_EINVAL;
    if (d->Sk == 0 && d->B > 0 && d->H > 0 && d->Sq > 0) return SF_EINVAL;
    return SF_OK;
}

}  // namespace

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
    return choose_splits(d);
}

extern "C" size_t sf_attn_workspace_bytes(const sf_attn_desc* d) {
    if (validate(d) != SF_OK) return 0;
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
    if (!q || !k || !v || !out) return SF_EINVAL;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out)) return SF_EINVAL;
    if (d->B > 65535 || d->H > 65535) return SF_ENOTSUP;

    const int ns = choose_splits(d);
    const int nqc = query_chunks(d);
    sfk::AttnArgs a{};
    a.q = static_cast<const uint16_t*>(q);
    a.k = static_cast<const uint16_t*>(k);
    a.v = static_cast<const uint16_t*>(v);
    a.o = out;
    a.valid_len = d->kv_valid_len;
    a.q_sb = d->q_stride[0]; a.q_sh = d->q_stride[1]; a.q_ss = d->q_stride[2];
    a.k_sb = d->k_stride[0]; a.k_sh = d->k_stride[1]; a.k_ss = d->k_stride[2];
    a.v_sb = d->v_stride[0]; a.v_sh = d->v_stride[1]; a.v_ss = d->v_stride[2];
    a.o_sb = d->o_stride[0]; a.o_sh = d->o_stride[1]; a.o_ss = d->o_stride[2];
    a.B = d->B; a.H = d->H; a.Sq = d->Sq; a.Sk = d->Sk;
    a.nsplit = ns;
    a.out_f32 = d->out_dtype == SF_F32;
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
    hipLaunchKernelGGL(sfk::attn_split_kernel, dim3(ns * nqc, d->H, d->B), dim3(sfk::kThreads), 0,
                       s, a);
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
        default: return "unknown status";
    }
}
