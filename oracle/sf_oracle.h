/*
 * sf_oracle.h — CPU restatement of servoflow's RDT-1B attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the MI355X
 * kernels: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.  The product (libsf_hip_kernels.so and the host code in
 * servoflow_amd/) never links, loads or falls back to it.
 *
 * Every function cites the reference file:line whose arithmetic it restates
 * (paths relative to the servoflow tree).  How each function is pinned
 * (golden vectors, known-answer tests, closed forms, invariants) is listed in
 * the test files under tests/ that exercise it.
 */
#ifndef SF_ORACLE_H_
#define SF_ORACLE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- deterministic inputs ------------------------------------------------ */
/* SplitMix64 -> Box-Muller N(0,1), `n` values, scaled by `std`. */
void sfo_randn(uint64_t seed, int64_t n, float std, float* out);
/* fp32 -> bf16 -> fp32, round to nearest even (what the GPU inputs hold). */
float sfo_bf16_round(float x);
void sfo_bf16_round_array(float* x, int64_t n);

/* ---- attention ------------------------------------------------------------
 * naive_attention_kernel, src/backend/cuda/ops/attention.cu:90-139: for each
 * (b, h, q) one online-softmax pass over the keys with fp32 running max m,
 * running sum and accumulator acc[D]; out = acc / sum.  scale == 0 means
 * 1/sqrt(D) (attention.cu:150); causal stops at key > q (attention.cu:117).
 * valid_len (NULL or B host ints) ignores keys >= valid_len[b]: the
 * reference's truncation of padded language (rdt1b.cpp:426).
 * Layout [B,H,S,D] contiguous, fp32. */
void sfo_attention_f32(const float* Q, const float* K, const float* V, float* O,
                       int B, int H, int Sq, int Sk, int D, float scale,
                       int causal, const int32_t* valid_len);

/* Same contraction in fp64 with a two-pass (max, then sum) softmax; an
 * independent evaluation order used to pin sfo_attention_f32. */
void sfo_attention_f64(const float* Q, const float* K, const float* V, double* O,
                       int B, int H, int Sq, int Sk, int D, double scale,
                       int causal, const int32_t* valid_len);

/* ---- normalisation ---------------------------------------------------------
 * rms_norm_kernel_impl, src/backend/cuda/ops/norm.cuh:89-122:
 * out = x * rsqrt(sum(x^2)/cols + eps) * gamma, fp32 accumulation. */
void sfo_rms_norm(const float* x, const float* gamma, float* out,
                  int64_t rows, int64_t cols, float eps);
/* fused_add_rms_norm_kernel, norm.cuh:130-171: residual += input, then
 * out = rms_norm(residual). */
void sfo_fused_add_rms_norm(const float* input, float* residual, const float* gamma,
                            float* out, int64_t rows, int64_t cols, float eps);

/* ---- activations: GeluOp / SiluOp, src/backend/cuda/ops/elementwise.cuh:35-68 */
float sfo_gelu_tanh(float x);
float sfo_silu(float x);

/* ---- linear: gemm_bias_act with trans_b (cuda_backend.cu:246-285, 337-467)
 * y[M,N] = act(x[M,K] . W[N,K]^T + bias[N]); act 0 none, 1 GELU(tanh), 2 SiLU.
 * fp32 accumulation in k order. */
void sfo_linear(const float* x, const float* W, const float* bias, float* y,
                int64_t M, int64_t N, int64_t K, int act);

/* ---- layout maps, src/backend/cuda/ops/split_ops.cuh ---------------------- */
/* split_qkv (:62-84): [B,S,3*H*D] -> Q,K,V [B,H,S,D] */
void sfo_split_qkv(const float* qkv, float* Q, float* K, float* V,
                   int B, int S, int H, int D);
/* split_kv (:210-226): [B,S,2*H*D] -> K,V [B,H,S,D] */
void sfo_split_kv(const float* kv, float* K, float* V, int B, int S, int H, int D);
/* seq_to_head (:123-137): [B,S,H*D] -> [B,H,S,D] */
void sfo_seq_to_head(const float* src, float* dst, int B, int S, int H, int D);
/* head_to_seq (:168-182): [B,H,S,D] -> [B,S,H*D] */
void sfo_head_to_seq(const float* src, float* dst, int B, int H, int S, int D);

/* ---- int8 weight dequant, src/backend/cuda/ops/quantization.cu:18-51 -------
 * out[i] = float(in[i]) * scale[i / K] (per_channel) or * scale[0]. */
void sfo_dequant_int8(const int8_t* in, const float* scale, float* out,
                      int64_t N, int64_t K, int per_channel);
/* Per-output-channel symmetric quantisation used to build the int8 weights:
 * s = max|W_row| / 127, q = clamp(rint(W / s), -127, 127). */
void sfo_quantize_int8_rows(const float* W, int64_t N, int64_t K, int8_t* q, float* scale);

/* ---- schedule, Schedule::linspace, src/sampling/flow_matching.cpp:10-17 --- */
void sfo_linspace(int num_steps, float t_start, float t_end, float* out);

/* ---- timestep embedding table, TimestepEmbedding::build_sincos_table,
 * src/models/rdt1b/dit_block.cu:58-72: table[step][i] = cos(step * f_i),
 * table[step][half + i] = sin(step * f_i), f_i = exp(-log(10000) * i / half),
 * all in float. ------------------------------------------------------------- */
void sfo_sincos_table(int max_steps, int freq_dim, float* table);
/* t in [0,1] -> integer timestep, rdt1b.cpp:312-313: round(t * (T - 1)) clamped. */
int sfo_timestep_index(float t, int num_train_timesteps);

#ifdef __cplusplus
}
#endif

#endif  /* SF_ORACLE_H_ */
