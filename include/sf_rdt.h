/*
 * sf_rdt.h — RDT-1B denoise-loop runtime on MI355X (libsf_rdt.so) and the
 * element-wise building blocks it uses (libsf_hip_kernels.so).
 *
 * The runtime is the native caller of the attention path: it owns the RDT-1B
 * weights, the per-inference cross-attention K/V cache and the hipGraph of
 * the fixed-shape Euler loop.  Reference interfaces it replaces (paths
 * relative to the servoflow tree):
 *   sf_rdt_set_condition     the condition half of RDT1BModel::encode_condition
 *                            (src/models/rdt1b/rdt1b.cpp:167-239) plus the
 *                            per-block K/V projection that
 *                            CrossAttention::forward repeats on every call
 *                            (src/models/rdt1b/dit_block.cu:288-308); here it
 *                            runs once per inference and is cached.
 *   sf_rdt_encode_condition  RDT1BModel::encode_condition: lang / img / state
 *                            adaptors (rdt1b.cpp:35-85, 167-239), then
 *                            sf_rdt_set_condition.
 *   sf_rdt_denoise_step      RDT1BModel::denoise_step (rdt1b.cpp:254-369,
 *                            IVLAModel::denoise_step,
 *                            include/servoflow/engine/inference_engine.h:83-87),
 *                            any batch size (the reference throws for B != 1,
 *                            rdt1b.cpp:268-270).
 *   sf_rdt_sample            FlowMatchingSampler::sample
 *                            (src/sampling/flow_matching.cpp:25-93): Euler
 *                            steps t_i = 1 - i/N, captured once into a
 *                            hipGraph and replayed.
 * All entry points return sf_status codes (sf_hip.h) and never throw.
 */
#ifndef SF_RDT_H_
#define SF_RDT_H_

#include <stddef.h>
#include <stdint.h>

#include "sf_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- element-wise building blocks (libsf_hip_kernels.so) ----------------- */

/* p[i] = N(0,1)(seed, i) * std as bf16 or fp32: a counter-based generator,
 * element i depends only on (seed, i).  Synthetic weight initialisation. */
int sf_init_normal(void* p, int32_t dtype, int64_t n, uint64_t seed, float std, void* stream);
int sf_fill_f32(float* p, int64_t n, float v, void* stream);
/* Rows of N(0,std)(seed, row*K + c) quantised per row: scale = max|w|/127,
 * q = clamp(rint(w/scale), -127, 127). */
int sf_init_int8_rows(int8_t* q, float* scale, int64_t N, int64_t K, uint64_t seed, float std,
                      void* stream);
/* out[r] = bf16([x_t[r], 1...1]) for rows of A actions: the state adaptor's
 * input cat(noisy_action, action_mask) (rdt1b.cpp:286-300). */
int sf_build_action_input(const float* x_t, void* out, int64_t rows, int32_t A, void* stream);
/* x[b] = [t_emb, f_emb, state[b], act[b, 0..T)] + pos (rdt1b.cpp:319-340);
 * x fp32 [B, T+3, D], state bf16 [B, D], act fp32 [B, T, D], pos fp32 [T+3, D]. */
int sf_assemble_tokens(float* x, const float* t_emb, const float* f_emb, const void* state,
                       const float* act, const float* pos, int32_t B, int32_t T, int32_t D,
                       void* stream);
/* out[b, l] = bf16(tok[b, l] + pos[l]) for l < L (rdt1b.cpp:342-349). */
int sf_add_pos_bf16(const void* tok, const float* pos, void* out, int32_t B, int32_t L, int32_t D,
                    void* stream);
/* x[b, t] += dt * v[b*S + 3 + t] (last T of S token rows; rdt1b.cpp:362,
 * flow_matching.cpp:77-78). */
int sf_euler_update(float* x, const float* v, int32_t B, int32_t T, int32_t A, int32_t S,
                    float dt, void* stream);
/* *out = max(*out, max |p[i]|) over n bf16 values (p 16-byte aligned; *out
 * fp32, >= 0, initialised by the caller, e.g. sf_fill_f32 with 0): NaN in p
 * gives NaN.  The runtime checks each layer's cached V against the fp16
 * range of the fast P.V form with it. */
int sf_absmax_bf16(const void* p, int64_t n, float* out, void* stream);
/* sf_absmax_bf16 over up to SF_ABSMAX_MAX_JOBS buffers in one launch, each
 * merged into its own *out (the runtime's per-layer V range check: one
 * launch instead of one per layer). */
#define SF_ABSMAX_MAX_JOBS 64
typedef struct sf_absmax_job {
    const void* p;   /* bf16, 16-byte aligned */
    int64_t n;
    float* out;
} sf_absmax_job;
int sf_absmax_bf16_batched(const sf_absmax_job* jobs, int32_t count, void* stream);
/* In place bf16 -> fp16 (round to nearest even) of every job's buffer whose
 * *out -- the max |x| sf_absmax_bf16_batched merged for the same job -- is
 * below `limit` (> 0, else SF_EINVAL; a NaN maximum is not below any
 * limit); the other buffers stay bf16.  The
 * runtime converts each layer's cached V this way with limit 65504, the
 * rule by which it picks the fp16 P.V form, so the attention reads fp16 V
 * (sf_attn_desc.v_f16) instead of converting every tile of every step. */
int sf_bf16_to_f16_below(const sf_absmax_job* jobs, int32_t count, float limit, void* stream);

/* ---- model runtime (libsf_rdt.so) ---------------------------------------- */

/* RDT1BConfig (include/servoflow/models/rdt1b/config.h:26-71) plus the batch
 * and weight format.  The reference's FFN has no expansion (config.h:60-61);
 * mlp_ratio > 1 builds the D -> mlp_ratio*D -> D variant (the "MLP 4x"
 * block of the benchmarked block-stack configuration, no reference
 * counterpart). */
typedef struct sf_rdt_config {
    int32_t hidden;              /* 2048 */
    int32_t layers;              /* 28 */
    int32_t heads;               /* 32 (head_dim 64) */
    int32_t action_dim;          /* 128 */
    int32_t horizon;             /* 64 action tokens; sequence = horizon + 3 */
    int32_t freq_dim;            /* 256 */
    int32_t state_dim;           /* 128 */
    int32_t lang_max;            /* 1024 padded language tokens */
    int32_t img_len;             /* 4374 image tokens */
    int32_t lang_token_dim;      /* 4096 (T5-XXL) */
    int32_t img_token_dim;       /* 1152 (SigLIP) */
    int32_t num_train_timesteps; /* 1000 */
    int32_t ctrl_freq;           /* 25 */
    int32_t num_steps;           /* 5 Euler steps */
    int32_t batch;
    int32_t int8_weights;        /* nonzero: block projections as int8 + fp32
                                    row scale.  At batch * (horizon + 3) > 160
                                    the runtime (int8 or not) also holds fp16
                                    copies of the block and final-layer
                                    matrices (2 bytes per weight), rewritten
                                    before the first pass after the parameters
                                    may have changed; with 2, no copy of the
                                    int8 matrices sf_gemm multiplies directly
                                    there (sf_gemm_int8_direct: every block
                                    matrix with K = 2048), which read their
                                    1-byte codes instead -- less memory and
                                    half the weight bytes, slower products */
    float eps;                   /* 1e-6 */
    int32_t mlp_ratio;           /* FFN hidden = mlp_ratio * hidden (1; 0 means 1) */
} sf_rdt_config;

typedef struct sf_rdt sf_rdt;

void sf_rdt_config_default(sf_rdt_config* cfg);
/* Allocates weights, caches and buffers on the current HIP device. */
int sf_rdt_create(const sf_rdt_config* cfg, sf_rdt** out);
void sf_rdt_destroy(sf_rdt* m);

/* Synthetic weights: matrices, biases and position embeddings ~ N(0, std),
 * RMSNorm gammas = 1 (the PyTorch init, test_rdt1b_alignment.py:76). */
int sf_rdt_init_random(sf_rdt* m, uint64_t seed, float std, void* stream);

/* Parameter table, named as the reference checkpoint keys. */
int32_t sf_rdt_num_params(const sf_rdt* m);
int sf_rdt_param_info(const sf_rdt* m, int32_t idx, const char** name, int32_t* dtype,
                      int32_t* ndim, int64_t shape[4]);
/* Device pointer to parameter idx.  The runtime multiplies fp16 copies of
 * some weights (above 160 projection rows, batch * 67, every block and
 * final-layer matrix but, with int8_weights = 2, the int8 ones read
 * directly; at most 160 rows with bf16 weights, the FFN matrices, whose
 * inputs are fp16); they are rebuilt before the first pass after this
 * call, after
 * sf_rdt_init_random / sf_rdt_load_safetensors, and after
 * sf_rdt_params_changed -- a caller that writes through a pointer it
 * obtained before a pass must call sf_rdt_params_changed before the next
 * one. */
void* sf_rdt_param_data(sf_rdt* m, int32_t idx);
/* Parameters were written through pointers from sf_rdt_param_data: the
 * weight copies are rebuilt (and sf_rdt_infer's cached condition
 * re-encoded) before the next pass. */
int sf_rdt_params_changed(sf_rdt* m);
float* sf_rdt_param_scale(sf_rdt* m, int32_t idx);      /* int8 row scales or NULL */
int32_t sf_rdt_find_param(const sf_rdt* m, const char* name);

/* Condition for the next inferences.  lang_c bf16 [B, lang_max, D],
 * lang_len int32 [B] (device; keys >= lang_len[b] are masked), img_c bf16
 * [B, img_len, D], state_tok bf16 [B, D]: the adaptor outputs.  Adds the
 * position embeddings and projects every block's cross-attention K/V once,
 * and embeds the control-frequency token and the timestep tokens of the
 * sampler's schedule (they depend on the weights only), so set or load the
 * weights before the condition. */
int sf_rdt_set_condition(sf_rdt* m, const void* lang_c, const int32_t* lang_len,
                         const void* img_c, const void* state_tok, void* stream);
/* Raw tokens: lang bf16 [B, lang_max, 4096], img bf16 [B, img_len, 1152],
 * state bf16 [B, state_dim]; runs the adaptors then sf_rdt_set_condition. */
int sf_rdt_encode_condition(sf_rdt* m, const void* lang_tokens, const int32_t* lang_len,
                            const void* img_tokens, const void* state, void* stream);
/* The language condition's token count L, 1..lang_max (default lang_max):
 * the length of the reference's language_tokens tensor [B, L, 4096]
 * (rdt1b.cpp:174-186), whose encode touches L rows, where the padded layout
 * here holds lang_max.  From the next condition set (sf_rdt_set_condition,
 * sf_rdt_encode_condition, or sf_rdt_infer, which re-encodes after a
 * change), the cross-attention reads at most L keys (lang_len[b] still
 * masks below that), and at batch 1 the language adaptor and every
 * language K/V projection run over the first L token rows only (batch > 1
 * keeps the padded rows: rows of one batch element are not contiguous with
 * the next one's).  Host only; prepares the new GEMM shapes (call outside
 * graph capture). */
int sf_rdt_set_lang_rows(sf_rdt* m, int32_t rows);

/* RDTBlock::forward (src/models/rdt1b/dit_block.cu:349-387) for blocks
 * [first, first + count) on the residual stream x fp32 [B, horizon+3, D]
 * (device, updated in place), with the cached condition. */
int sf_rdt_run_blocks(sf_rdt* m, float* x, int32_t first, int32_t count, void* stream);

/* velocity[B, T, A] = v(x_t, t) for fp32 device buffers. */
int sf_rdt_denoise_step(sf_rdt* m, const float* x_t, float t, float* velocity, void* stream);

/* x[B, T, A] (fp32, device) <- num_steps Euler steps from t = 1 to 0.
 * use_graph != 0 captures the loop into a hipGraph on the first call and
 * replays it afterwards (inputs are copied in and out around the graph). */
int sf_rdt_sample(sf_rdt* m, float* x, int32_t use_graph, void* stream);

/* InferenceEngine::infer (src/engine/inference_engine.cpp:99-175) on this
 * runtime: (1) sf_rdt_encode_condition on the raw tokens when frame_id
 * differs from the frame of the cached condition, or when none is cached
 * (first call, or a condition set with sf_rdt_set_condition /
 * sf_rdt_encode_condition, or weights changed since) -- the reference's
 * mark_new_frame / frame-id test (:106-128); otherwise the token pointers
 * are not read; (2) x_T [B, T, A] ~ N(0,1) from noise_seed, element i from
 * (noise_seed, i) as sf_init_normal, or zeros for noise_seed == 0 (the
 * reference's placeholder, :133-136); (3) the Euler loop as one hipGraph
 * replay (sf_rdt_sample); (4) the action chunk, fp32 [B, T, A], copied to
 * the HOST buffer action_out, and the stream synchronised before returning
 * (decode_action is the identity for RDT-1B, rdt1b.h:35-37).  *encoded
 * (optional) is set to 1 when the condition was encoded by this call. */
int sf_rdt_infer(sf_rdt* m, uint64_t frame_id, const void* lang_tokens, const int32_t* lang_len,
                 const void* img_tokens, const void* state, uint64_t noise_seed,
                 float* action_out, int32_t* encoded, void* stream);

/* P.V form block `layer`'s cross-attention runs with the current condition:
 * 0 the fp16 form (every cached V element below 65504 in magnitude), 1 the
 * exact bf16 form (a larger, infinite or NaN element), -1 on error.  The
 * runtime measures each layer's max |V| when a condition is set and chooses
 * the form before the next step or graph capture (one wait for the
 * condition's encode per new condition); asking here does the same. */
int32_t sf_rdt_pv_exact(sf_rdt* m, int32_t layer);

/* Cross-attention K or V cache of block `layer` ([B, H, S, 64]): K in
 * bf16; V in fp16 when the layer runs the fp16 P.V form
 * (sf_rdt_pv_exact == 0: converted once when the condition was set), else
 * bf16. */
void* sf_rdt_cache_ptr(sf_rdt* m, int32_t layer, int32_t which_v);

/* ---- checkpoints (safetensors) ------------------------------------------- */

/* One tensor of a safetensors file (SafeTensorsLoader::TensorMeta,
 * include/servoflow/loader/safetensors.h; header format of
 * src/loader/safetensors.cpp:75-105).  data_begin / data_end are absolute
 * byte offsets in the file; dtype is an sf_dtype value or -1. */
typedef struct sf_st_entry {
    char name[256];
    int32_t dtype;
    int32_t ndim;
    int64_t shape[8];
    uint64_t data_begin, data_end;
} sf_st_entry;

/* Lists the tensors of a safetensors file (SafeTensorsLoader::inspect,
 * safetensors.cpp:110-114): fills up to max_entries entries and sets *count
 * to the number of tensors in the file.  Host only. */
int sf_safetensors_inspect(const char* path, sf_st_entry* entries, int32_t max_entries,
                           int32_t* count);

#define SF_LOAD_PARTIAL 1   /* do not fail when a model parameter is absent */

/* Loads a checkpoint into the parameter table (SafeTensorsLoader::load +
 * load_weight_from_map, safetensors.cpp:117-190): names as the servoflow
 * checkpoint keys, HuggingFace names accepted through remap_key
 * (tools/convert/hf_to_servoflow.py:41-65: leading "model." dropped, EMA and
 * optimizer entries skipped); F32 / F16 / BF16 tensors converted to the
 * parameter's type (bf16 round-to-nearest-even, or int8 rows quantised
 * scale = max|w| / 127 in int8 mode); shapes must match up to leading 1s.
 * Keys the model does not have are ignored; a model parameter absent from
 * the file is an error unless flags has SF_LOAD_PARTIAL.  *loaded = number of
 * parameters written.  Synchronous (hipMemcpy); sf_rdt_last_error describes
 * a failure. */
int sf_rdt_load_safetensors(sf_rdt* m, const char* path, int32_t flags, int32_t* loaded);

/* Message of the last failure of a call on m ("" if none). */
const char* sf_rdt_last_error(const sf_rdt* m);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* SF_RDT_H_ */
