/*
 * sf_oracle.c — CPU restatement of servoflow's RDT-1B attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the MI355X kernels, loaded by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, never by
 * the product.  Each function cites the reference file:line it restates.
 * Built with -ffp-contract=off so every multiply-add rounds as written.
 */
#include "sf_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- deterministic inputs ------------------------------------------------ */

/* SplitMix64 (Steele, Lea, Flood 2014): state += golden gamma, then the
 * variant-13 finaliser. */
static uint64_t splitmix64_next(uint64_t* s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void sfo_randn(uint64_t seed, int64_t n, float std, float* out) {
    uint64_t s = seed;
    const double two_pi = 6.283185307179586476925286766559;
    const double inv53 = 1.0 / 9007199254740992.0; /* 2^-53 */
    for (int64_t i = 0; i < n; i += 2) {
        const double u1 = ((double)(splitmix64_next(&s) >> 11) + 1.0) * inv53; /* (0,1] */
        const double u2 = (double)(splitmix64_next(&s) >> 11) * inv53;         /* [0,1) */
        const double rad = sqrt(-2.0 * log(u1));
        out[i] = (float)(rad * cos(two_pi * u2)) * std;
        if (i + 1 < n) out[i + 1] = (float)(rad * sin(two_pi * u2)) * std;
    }
}

float sfo_bf16_round(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        u |= 0x00400000u;
        u &= 0xffff0000u;
    } else {
        u += 0x7fffu + ((u >> 16) & 1u);
        u &= 0xffff0000u;
    }
    float y;
    memcpy(&y, &u, 4);
    return y;
}

void sfo_bf16_round_array(float* x, int64_t n) {
    for (int64_t i = 0; i < n; ++i) x[i] = sfo_bf16_round(x[i]);
}

/* ---- attention ----------------------------------------------------------- */

static int eff_keys(int Sk, const int32_t* valid_len, int b) {
    if (!valid_len) return Sk;
    int v = valid_len[b];
    return v < 0 ? 0 : (v > Sk ? Sk : v);
}

/* naive_attention_kernel, attention.cu:90-139 (one query per iteration). */
void sfo_attention_f32(const float* Q, const float* K, const float* V, float* O,
                       int B, int H, int Sq, int Sk, int D, float scale,
                       int causal, const int32_t* valid_len) {
    if (scale == 0.f) scale = 1.f / sqrtf((float)D);
    const int64_t BH = (int64_t)B * H;
#pragma omp parallel for schedule(static)
    for (int64_t bh = 0; bh < BH; ++bh) {
        const int b = (int)(bh / H);
        const int nk = eff_keys(Sk, valid_len, b);
        float* acc = (float*)malloc(sizeof(float) * (size_t)D);
        const float* Kbh = K + bh * (int64_t)Sk * D;
        const float* Vbh = V + bh * (int64_t)Sk * D;
        for (int q = 0; q < Sq; ++q) {
            const float* Qr = Q + (bh * Sq + q) * (int64_t)D;
            float m = -1e30f, sum = 0.f;
            for (int d = 0; d < D; ++d) acc[d] = 0.f;
            for (int k = 0; k < nk; ++k) {
                if (causal && k > q) break;                       /* :117 */
                float dot = 0.f;
                for (int d = 0; d < D; ++d) dot += Qr[d] * Kbh[(int64_t)k * D + d];
                dot *= scale;
                const float new_m = fmaxf(m, dot);                /* :125 */
                const float exp_old = expf(m - new_m);
                const float exp_new = expf(dot - new_m);
                for (int d = 0; d < D; ++d)
                    acc[d] = acc[d] * exp_old + exp_new * Vbh[(int64_t)k * D + d];
                sum = sum * exp_old + exp_new;
                m = new_m;
            }
            /* :136-138; an empty key set (valid_len 0) gives zeros here, the
             * convention sf_attn_fwd documents. */
            const float inv = sum > 0.f ? 1.f / sum : 0.f;
            float* Or = O + (bh * Sq + q) * (int64_t)D;
            for (int d = 0; d < D; ++d) Or[d] = acc[d] * inv;
        }
        free(acc);
    }
}

void sfo_attention_f64(const float* Q, const float* K, const float* V, double* O,
                       int B, int H, int Sq, int Sk, int D, double scale,
                       int causal, const int32_t* valid_len) {
    if (scale == 0.0) scale = 1.0 / sqrt((double)D);
    const int64_t BH = (int64_t)B * H;
#pragma omp parallel for schedule(static)
    for (int64_t bh = 0; bh < BH; ++bh) {
        const int b = (int)(bh / H);
        const int nk = eff_keys(Sk, valid_len, b);
        double* sc = (double*)malloc(sizeof(double) * (size_t)(nk > 0 ? nk : 1));
        const float* Kbh = K + bh * (int64_t)Sk * D;
        const float* Vbh = V + bh * (int64_t)Sk * D;
        for (int q = 0; q < Sq; ++q) {
            const float* Qr = Q + (bh * Sq + q) * (int64_t)D;
            const int kn = causal ? (q + 1 < nk ? q + 1 : nk) : nk;
            double mx = -INFINITY;
            for (int k = 0; k < kn; ++k) {
                double dot = 0.0;
                for (int d = 0; d < D; ++d) dot += (double)Qr[d] * (double)Kbh[(int64_t)k * D + d];
                sc[k] = dot * scale;
                if (sc[k] > mx) mx = sc[k];
            }
            double den = 0.0;
            for (int k = 0; k < kn; ++k) {
                sc[k] = exp(sc[k] - mx);
                den += sc[k];
            }
            double* Or = O + (bh * Sq + q) * (int64_t)D;
            for (int d = 0; d < D; ++d) {
                double num = 0.0;
                for (int k = 0; k < kn; ++k) num += sc[k] * (double)Vbh[(int64_t)k * D + d];
                Or[d] = den > 0.0 ? num / den : 0.0;
            }
        }
        free(sc);
    }
}

/* ---- normalisation ------------------------------------------------------- */

/* rms_norm_kernel_impl, norm.cuh:89-122. */
void sfo_rms_norm(const float* x, const float* gamma, float* out,
                  int64_t rows, int64_t cols, float eps) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + r * cols;
        float ss = 0.f;
        for (int64_t c = 0; c < cols; ++c) ss += xr[c] * xr[c];
        const float inv_rms = 1.f / sqrtf(ss / (float)cols + eps);
        float* orow = out + r * cols;
        for (int64_t c = 0; c < cols; ++c) orow[c] = xr[c] * inv_rms * gamma[c];
    }
}

/* fused_add_rms_norm_kernel, norm.cuh:130-171 (residual kept in fp32). */
void sfo_fused_add_rms_norm(const float* input, float* residual, const float* gamma,
                            float* out, int64_t rows, int64_t cols, float eps) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        float* res = residual + r * cols;
        const float* in = input + r * cols;
        float ss = 0.f;
        for (int64_t c = 0; c < cols; ++c) {
            const float v = in[c] + res[c];
            res[c] = v;
            ss += v * v;
        }
        const float inv_rms = 1.f / sqrtf(ss / (float)cols + eps);
        float* orow = out + r * cols;
        for (int64_t c = 0; c < cols; ++c) orow[c] = res[c] * inv_rms * gamma[c];
    }
}

/* ---- activations, elementwise.cuh:35-68 ---------------------------------- */

float sfo_gelu_tanh(float x) {
    const float kAlpha = 0.7978845608028654f; /* sqrt(2/pi) */
    const float kBeta = 0.044715f;
    const float t = tanhf(kAlpha * (x + kBeta * x * x * x));
    return 0.5f * x * (1.f + t);
}

float sfo_silu(float x) { return x / (1.f + expf(-x)); }

/* ---- linear --------------------------------------------------------------- */

/* y = act(x . W^T + bias).  The k loop keeps 8 independent fp32 partial sums
 * (k mod 8) that are added pairwise at the end: a fixed order that the
 * compiler can vectorise without reassociating anything. */
void sfo_linear(const float* x, const float* W, const float* bias, float* y,
                int64_t M, int64_t N, int64_t K, int act) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t n = 0; n < N; ++n) {
            const float* xr = x + m * K;
            const float* wr = W + n * K;
            float p[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            int64_t k = 0;
            for (; k + 8 <= K; k += 8)
                for (int j = 0; j < 8; ++j) p[j] += xr[k + j] * wr[k + j];
            for (; k < K; ++k) p[k & 7] += xr[k] * wr[k];
            float acc = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
            if (bias) acc += bias[n];
            if (act == 1) acc = sfo_gelu_tanh(acc);
            else if (act == 2) acc = sfo_silu(acc);
            y[m * N + n] = acc;
        }
    }
}

/* ---- layout maps, split_ops.cuh ------------------------------------------ */

void sfo_split_qkv(const float* qkv, float* Q, float* K, float* V, int B, int S, int H, int D) {
    const int64_t total = (int64_t)B * H * S * D;
    for (int64_t idx = 0; idx < total; ++idx) {
        const int64_t b = idx / ((int64_t)H * S * D);
        const int64_t h = (idx / ((int64_t)S * D)) % H;
        const int64_t s = (idx / D) % S;
        const int64_t d = idx % D;
        const int64_t src = b * S * 3 * H * D + s * 3 * H * D;
        Q[idx] = qkv[src + (0 * H + h) * D + d];
        K[idx] = qkv[src + (1 * H + h) * D + d];
        V[idx] = qkv[src + (2 * H + h) * D + d];
    }
}

void sfo_split_kv(const float* kv, float* K, float* V, int B, int S, int H, int D) {
    const int64_t total = (int64_t)B * H * S * D;
    for (int64_t idx = 0; idx < total; ++idx) {
        const int64_t b = idx / ((int64_t)H * S * D);
        const int64_t h = (idx / ((int64_t)S * D)) % H;
        const int64_t s = (idx / D) % S;
        const int64_t d = idx % D;
        const int64_t src = b * S * 2 * H * D + s * 2 * H * D;
        K[idx] = kv[src + (0 * H + h) * D + d];
        V[idx] = kv[src + (1 * H + h) * D + d];
    }
}

void sfo_seq_to_head(const float* src, float* dst, int B, int S, int H, int D) {
    const int64_t total = (int64_t)B * H * S * D;
    for (int64_t idx = 0; idx < total; ++idx) {
        const int64_t b = idx / ((int64_t)H * S * D);
        const int64_t h = (idx / ((int64_t)S * D)) % H;
        const int64_t s = (idx / D) % S;
        const int64_t d = idx % D;
        dst[idx] = src[b * S * H * D + s * H * D + h * D + d];
    }
}

void sfo_head_to_seq(const float* src, float* dst, int B, int H, int S, int D) {
    const int64_t total = (int64_t)B * H * S * D;
    for (int64_t idx = 0; idx < total; ++idx) {
        const int64_t b = idx / ((int64_t)H * S * D);
        const int64_t h = (idx / ((int64_t)S * D)) % H;
        const int64_t s = (idx / D) % S;
        const int64_t d = idx % D;
        dst[b * S * H * D + s * H * D + h * D + d] = src[idx];
    }
}

/* ---- int8 ----------------------------------------------------------------- */

/* dequantize_int8_fp16_kernel, quantization.cu:18-51 (row = i / K). */
void sfo_dequant_int8(const int8_t* in, const float* scale, float* out,
                      int64_t N, int64_t K, int per_channel) {
    const int64_t n = N * K;
    for (int64_t i = 0; i < n; ++i) {
        const float s = per_channel ? scale[i / K] : scale[0];
        out[i] = (float)in[i] * s;
    }
}

void sfo_quantize_int8_rows(const float* W, int64_t N, int64_t K, int8_t* q, float* scale) {
    for (int64_t r = 0; r < N; ++r) {
        float amax = 0.f;
        for (int64_t c = 0; c < K; ++c) {
            const float a = fabsf(W[r * K + c]);
            if (a > amax) amax = a;
        }
        const float s = amax > 0.f ? amax / 127.f : 1.f;
        scale[r] = s;
        for (int64_t c = 0; c < K; ++c) {
            float v = rintf(W[r * K + c] / s);
            if (v > 127.f) v = 127.f;
            if (v < -127.f) v = -127.f;
            q[r * K + c] = (int8_t)v;
        }
    }
}

/* ---- schedule, flow_matching.cpp:10-17 ----------------------------------- */

void sfo_linspace(int num_steps, float t_start, float t_end, float* out) {
    for (int i = 0; i <= num_steps; ++i) {
        const float alpha = (float)i / (float)num_steps;
        out[i] = t_start + alpha * (t_end - t_start);
    }
}

/* ---- timestep embedding, dit_block.cu:58-72 and rdt1b.cpp:312-313 --------- */

void sfo_sincos_table(int max_steps, int freq_dim, float* table) {
    const float max_period = 10000.f;
    const int half = freq_dim / 2;
    for (int step = 0; step < max_steps; ++step) {
        const float t = (float)step;
        for (int i = 0; i < half; ++i) {
            const float freq = expf(-logf(max_period) * (float)i / (float)half);
            const float angle = t * freq;
            table[(int64_t)step * freq_dim + i] = cosf(angle);
            table[(int64_t)step * freq_dim + half + i] = sinf(angle);
        }
    }
}

int sfo_timestep_index(float t, int num_train_timesteps) {
    long v = lroundf(t * (float)(num_train_timesteps - 1));
    if (v < 0) v = 0;
    if (v > num_train_timesteps - 1) v = num_train_timesteps - 1;
    return (int)v;
}
