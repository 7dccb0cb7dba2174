// RDT-1B denoise-loop runtime for MI355X (libsf_rdt.so).
//
// Native restatement of the reference's model and sampler layers:
//   RDT1BModel (src/models/rdt1b/rdt1b.cpp), RDTBlock / SelfAttention /
//   CrossAttention / Mlp / TimestepEmbedding / FinalLayer
//   (src/models/rdt1b/dit_block.cu), FlowMatchingSampler
//   (src/sampling/flow_matching.cpp).
// Differences by design (MI355X-first):
//   * every buffer (weights, residual stream, per-head q/k/v, the
//     per-inference cross-attention K/V cache, attention workspace) is
//     allocated once at creation from one device arena, so the step issues
//     no allocation and is capturable (the reference calls cudaMallocAsync in
//     every op, cuda_backend.cu:51-62, 490);
//   * the block is a short chain of fused kernels (sf_hip.h) instead of
//     ~25 launches: the QKV projection writes normed per-head Q/K/V,
//     attention writes [B,S,H*64] directly, and each branch projection adds
//     into the fp32 residual and applies the next RMSNorm in its epilogue
//     (proj -> norm2, cross proj -> norm3, fc2 -> next block's norm1 or the
//     final norm), so no standalone norm runs inside the block stack;
//   * the cross-attention K/V projection runs once per inference
//     (sf_rdt_set_condition) instead of in every block call
//     (dit_block.cu:288-293);
//   * batch > 1 is supported (rdt1b.cpp:268-270 throws).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <algorithm>
#include <array>
#include <cstring>
#include <string>
#include <vector>

#include "sf_hip.h"
#include "sf_rdt.h"
#include "rdt_internal.h"

namespace {

#define SF_TRY(expr)                       \
    do {                                   \
        const int _st = (expr);            \
        if (_st != SF_OK) return _st;      \
    } while (0)

#define SF_HIP(expr)                                 \
    do {                                             \
        if ((expr) != hipSuccess) return SF_EDEVICE; \
    } while (0)

struct Param {
    std::string name;
    int32_t dtype = SF_BF16;
    std::vector<int64_t> shape;
    bool ones = false;          // RMSNorm gamma
    size_t offset = 0;          // into the arena
    size_t scale_offset = 0;    // int8 row scales
    void* data = nullptr;
    float* scale = nullptr;
    int64_t numel() const {
        int64_t n = 1;
        for (int64_t s : shape) n *= s;
        return n;
    }
    size_t bytes() const {
        return (size_t)numel() * (dtype == SF_F32 ? 4 : dtype == SF_BF16 ? 2 : 1);
    }
};

struct LayerIdx {
    int norm1, norm2, norm3;
    int qkv_w, qkv_b, q_norm, k_norm, proj_w, proj_b;
    int cq_w, cq_b, ckv_w, ckv_b, cq_norm, ck_norm, cproj_w, cproj_b;
    int fc1_w, fc1_b, fc2_w, fc2_b;
};

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// The projection weights a block's forward multiplies by.
std::array<int, 6> block_weights(const LayerIdx& L) {
    return {L.qkv_w, L.proj_w, L.cq_w, L.cproj_w, L.fc1_w, L.fc2_w};
}

}  // namespace

struct sf_rdt {
    sf_rdt_config cfg{};
    std::vector<Param> params;
    std::vector<LayerIdx> layers;
    int sa[6], la[4], ia[4], te[4], fe[4];
    int xpos, lpos, ipos, fnorm, f1w, f1b, f2w, f2b;

    char* arena = nullptr;
    size_t arena_bytes = 0;
    hipStream_t own_stream = nullptr;

    // activations (batch B, sequence S = horizon + 3)
    float* x = nullptr;            // [B*S, D] fp32 residual stream
    uint16_t* n = nullptr;         // [B*S, D] bf16 norm1 / norm2 / final-norm output
    uint16_t *q = nullptr, *k = nullptr, *v = nullptr;   // [B, H, S, 64]
    // Above 160 rows (the library-path GEMMs) the QKV projection is kept as
    // its bf16 output [B*S, 3D] and the cross-q projection's as [B*S, D] in
    // q; the attention reads Q / K / V from those rows and applies q_norm /
    // k_norm as it loads them (sf_attn_desc.q_gamma / k_gamma) in place of
    // the per-head epilogue pass.
    bool rows_qkv = false;
    uint16_t* qkv_rows = nullptr;
    uint16_t* a = nullptr;         // [B*S, D] attention output (act16)
    // Element type of the projections' 16-bit inputs.  The FFN's inputs
    // (norm3 output, GELU hidden; ffn_dtype) are fp16 at every batch size
    // (3 more significant bits than bf16 at the same bytes; of the block's
    // 16-bit storage points these two move the block output furthest from
    // fp32 arithmetic); on the split-K path the fc1 / fc2 weight fragments
    // are converted to fp16 in registers.  The other inputs -- norm1 /
    // norm2 / final-norm outputs and attention outputs (act16) -- are bf16
    // while B*S rows fit the split-K regime (<= 160) and fp16 above it,
    // where the library path multiplies fp16 activations by fp16 copies of
    // the weights (w16) and keeps its 16-bit products in fp16: with bf16
    // inputs and bf16 products a block sat at 1.6-1.8e-3 from fp32
    // arithmetic, with fp16 ones at 0.6-0.8e-3.  fp16 holds magnitudes below
    // 65504: norm outputs stay below sqrt(hidden) * max|gamma|, attention
    // outputs below max|V| (the cross K/V cache's range is checked when the
    // condition is set), products and GELU outputs of the block below it as
    // long as the model's activations do.
    int32_t ffn_dtype = SF_F16;
    int32_t act16 = SF_BF16;
    // Deferred RMSNorm (split-K regime, B*S <= 160): the norm1 / norm2
    // producers -- the entry norm, the fc2 and attention-proj residual adds --
    // store x * gamma and per-64-column sums of squares (row_ss, [D/64][B*S])
    // and the consumers (the QKV and cross-q projections, or the language
    // attention finishing Q from partials) apply the row's 1/rms after their
    // contraction: every CU takes part in the residual-add kernels, which
    // otherwise run one workgroup per row.  norm3 and the final norm keep the
    // row-wide form (their fp16 outputs need the normalised range).
    // n_deferred: whether n holds deferred rows (set as kernels are enqueued).
    bool defer = false;
    bool n_deferred = false;
    float* row_ss = nullptr;
    void* n3 = nullptr;            // [B*S, D] norm3 output
    void* h = nullptr;             // [B*S, F] FFN hidden
    uint16_t* act_in = nullptr;    // [B*T, 2A]
    uint16_t *sa0 = nullptr, *sa1 = nullptr;   // [B*T, D]
    float* act_out = nullptr;      // [B*T, D]
    uint16_t* sincos = nullptr;    // [num_train_timesteps, freq_dim] bf16
    uint16_t* emb_h = nullptr;     // [1, D]
    float* t_emb = nullptr;        // [D]
    // the timestep tokens of the sampler's schedule, [num_steps][D],
    // embedded with the condition (they depend on the weights and the step
    // index only), read by the sampled loop instead of re-embedding
    float* t_emb_steps = nullptr;
    float* f_emb = nullptr;        // [D]
    uint16_t* state_tok = nullptr; // [B, D]
    float* vel_rows = nullptr;     // [B*S, A]
    float* x_state = nullptr;      // [B*T*A] sampler state
    int32_t* lang_len = nullptr;   // [B]
    uint16_t* lang_c = nullptr;    // [B, lang_max, D] condition tokens + pos
    uint16_t* img_c = nullptr;     // [B, img_len, D]
    uint16_t* ad_h = nullptr;      // adaptor hidden [B*max(Lmax, I), D]
    std::vector<uint16_t*> ck, cv; // per-layer cross K/V cache [B, H, Sc, 64]
    // The K/V projections of the blocks that attend to one condition (group
    // 0: language, even blocks; 1: image, odd blocks), laid out back to back
    // in the arena -- weights, then biases, then int8 row scales, in block
    // order -- so that one GEMM of N = blocks * 2D computes all of them
    // when the rows run on the library path and the product fits kv_prod
    // (sf_heads_bf16 then splits it per block).
    struct KvGroup {
        std::vector<int> blocks;
        const void* W = nullptr;       // [blocks * 2D][D]
        const float* bias = nullptr;   // [blocks * 2D]
        const float* scale = nullptr;  // int8 row scales or null
        int32_t w_dtype = SF_BF16;
        bool contiguous = false;
        int rows_max = 0;              // condition rows of one set (batch 1: L <= lang_max)
    } kvg[2];
    uint16_t* kv_prod = nullptr;   // [rows][blocks * 2D] bf16 product of a batched group
    size_t kv_prod_bytes = 0;
    // Language blocks at <= 160 rows: the cross-q projection leaves its
    // split-K partials (SF_EPI_PARTIALS) and the language attention, on its
    // query-block grid, finishes Q from them (sum, scale, bias, q_norm) --
    // one launch less per language block.  cq_splits: the partials' count.
    int cq_splits = 0;
    void* attn_ws = nullptr;
    size_t attn_ws_bytes = 0;
    void* gemm_ws = nullptr;       // split-K partial sums, shared by the stream's GEMMs
    size_t gemm_ws_bytes = 0;
    // fp16 copies of projection weights (w16_params: above 160 rows every
    // block's six and the final layer's two; at most 160 rows with bf16
    // weights the ones multiplying fp16 inputs; int8 codes widened exactly,
    // bf16 weights rounded to fp16; sf_weights_to_f16, up to eight
    // matrices per launch), made before the first pass and again before
    // the first pass after the parameters may have changed (w16_stale), on
    // the pass's stream and outside any graph capture -- not once per loop:
    // a batch-16 loop refreshing them in its graph took 0.8 ms more.
    // codes16_of[param] is a weight's copy (fixed at creation).
    char* codes16 = nullptr;
    size_t codes16_bytes = 0;
    std::vector<const void*> codes16_of;
    // The copies may no longer match the weights: set by every call that
    // writes parameters or hands out a pointer to them (and by
    // sf_rdt_params_changed), cleared by the refresh at the start of the
    // next pass.
    bool w16_stale = true;

    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
    hipStream_t graph_stream = nullptr;

    // P.V form of each block's cross-attention.  The fast fp16 form holds a
    // cached V element only below 65504 in magnitude; sf_rdt_set_condition
    // measures each layer's max |V| on the device, and before the next step
    // (or graph capture) the host reads it once and runs a layer whose V
    // would overflow (or holds NaN/inf) in the exact bf16 form.
    float* v_absmax = nullptr;        // [layers] device
    float* v_absmax_host = nullptr;   // [layers] pinned host copy
    hipEvent_t cond_event = nullptr;  // recorded after the copy
    uint64_t cond_gen = 0;            // conditions set so far
    uint64_t forms_gen = 0;           // condition the forms were chosen for
    std::vector<uint8_t> exact_pv;    // [layers]

    // sf_rdt_infer's condition cache: the frame id the cached condition was
    // encoded for, valid until another condition or new weights replace it
    float* x_infer = nullptr;      // [B*T*A] initial noise, then the action chunk
    bool infer_cond_valid = false;

    // Language token rows per batch element (the reference's L, the length
    // of its language_tokens tensor): lang_rows is the caller's setting,
    // cond_lang_rows the value the cached condition was encoded with (the
    // cross-attention reads at most that many keys).  At batch 1 the
    // language adaptor and K/V projections run over those rows only.
    int32_t lang_rows = 0;
    int32_t cond_lang_rows = 0;
    uint64_t infer_cond_frame = 0;

    std::string last_error;
};

void sf_rdt_set_error(sf_rdt* m, const std::string& msg) {
    if (m) m->last_error = msg;
}

void sf_rdt_weights_changed(sf_rdt* m) {
    if (!m) return;
    m->infer_cond_valid = false;
    m->w16_stale = true;
}

extern "C" const char* sf_rdt_last_error(const sf_rdt* m) { return m ? m->last_error.c_str() : ""; }

namespace {

int add_param(sf_rdt* m, const std::string& name, int32_t dtype, std::vector<int64_t> shape,
              bool ones = false) {
    Param p;
    p.name = name;
    p.dtype = dtype;
    p.shape = std::move(shape);
    p.ones = ones;
    m->params.push_back(std::move(p));
    return (int)m->params.size() - 1;
}

// Projection weight [N, K]: bf16, or int8 + fp32 row scale in int8 mode.
int add_matrix(sf_rdt* m, const std::string& name, int64_t N, int64_t K, bool quantisable) {
    const bool i8 = quantisable && m->cfg.int8_weights;
    return add_param(m, name, i8 ? SF_I8 : SF_BF16, {N, K});
}

int64_t ffn_dim(const sf_rdt_config& c) {
    return (int64_t)(c.mlp_ratio > 1 ? c.mlp_ratio : 1) * c.hidden;
}

void build_param_table(sf_rdt* m) {
    const sf_rdt_config& c = m->cfg;
    const int64_t D = c.hidden;
    auto vec = [&](const std::string& nm, int64_t n, bool ones = false) {
        return add_param(m, nm, SF_F32, {n}, ones);
    };
    // adaptors (rdt1b.cpp:117-126; mlp2x/mlp3x keys "0", "2", "4")
    m->la[0] = add_matrix(m, "lang_adaptor.0.weight", D, c.lang_token_dim, false);
    m->la[1] = vec("lang_adaptor.0.bias", D);
    m->la[2] = add_matrix(m, "lang_adaptor.2.weight", D, D, false);
    m->la[3] = vec("lang_adaptor.2.bias", D);
    m->ia[0] = add_matrix(m, "img_adaptor.0.weight", D, c.img_token_dim, false);
    m->ia[1] = vec("img_adaptor.0.bias", D);
    m->ia[2] = add_matrix(m, "img_adaptor.2.weight", D, D, false);
    m->ia[3] = vec("img_adaptor.2.bias", D);
    m->sa[0] = add_matrix(m, "state_adaptor.0.weight", D, 2 * c.state_dim, false);
    m->sa[1] = vec("state_adaptor.0.bias", D);
    m->sa[2] = add_matrix(m, "state_adaptor.2.weight", D, D, false);
    m->sa[3] = vec("state_adaptor.2.bias", D);
    m->sa[4] = add_matrix(m, "state_adaptor.4.weight", D, D, false);
    m->sa[5] = vec("state_adaptor.4.bias", D);
    // timestep / control-frequency embedders (dit_block.cu:84-100)
    m->te[0] = add_matrix(m, "t_embedder.mlp.0.weight", D, c.freq_dim, false);
    m->te[1] = vec("t_embedder.mlp.0.bias", D);
    m->te[2] = add_matrix(m, "t_embedder.mlp.2.weight", D, D, false);
    m->te[3] = vec("t_embedder.mlp.2.bias", D);
    m->fe[0] = add_matrix(m, "freq_embedder.mlp.0.weight", D, c.freq_dim, false);
    m->fe[1] = vec("freq_embedder.mlp.0.bias", D);
    m->fe[2] = add_matrix(m, "freq_embedder.mlp.2.weight", D, D, false);
    m->fe[3] = vec("freq_embedder.mlp.2.bias", D);
    // position embeddings (rdt1b.cpp:133-135)
    m->xpos = add_param(m, "x_pos_embed", SF_F32, {1, c.horizon + 3, D});
    m->lpos = add_param(m, "lang_cond_pos_embed", SF_F32, {1, c.lang_max, D});
    m->ipos = add_param(m, "img_cond_pos_embed", SF_F32, {1, c.img_len, D});
    // blocks (dit_block.cu:168-183, 243-260, 331-347)
    m->layers.resize(c.layers);
    for (int i = 0; i < c.layers; ++i) {
        const std::string p = "blocks." + std::to_string(i) + ".";
        LayerIdx& L = m->layers[i];
        L.norm1 = vec(p + "norm1.weight", D, true);
        L.norm2 = vec(p + "norm2.weight", D, true);
        L.norm3 = vec(p + "norm3.weight", D, true);
        L.qkv_w = add_matrix(m, p + "attn.qkv.weight", 3 * D, D, true);
        L.qkv_b = vec(p + "attn.qkv.bias", 3 * D);
        L.q_norm = vec(p + "attn.q_norm.weight", 64, true);
        L.k_norm = vec(p + "attn.k_norm.weight", 64, true);
        L.proj_w = add_matrix(m, p + "attn.proj.weight", D, D, true);
        L.proj_b = vec(p + "attn.proj.bias", D);
        L.cq_w = add_matrix(m, p + "cross_attn.q.weight", D, D, true);
        L.cq_b = vec(p + "cross_attn.q.bias", D);
        L.ckv_w = add_matrix(m, p + "cross_attn.kv.weight", 2 * D, D, true);
        L.ckv_b = vec(p + "cross_attn.kv.bias", 2 * D);
        L.cq_norm = vec(p + "cross_attn.q_norm.weight", 64, true);
        L.ck_norm = vec(p + "cross_attn.k_norm.weight", 64, true);
        L.cproj_w = add_matrix(m, p + "cross_attn.proj.weight", D, D, true);
        L.cproj_b = vec(p + "cross_attn.proj.bias", D);
        // FFN D -> F -> D, F = mlp_ratio * D (the reference: F = D,
        // config.h:60-61, dit_block.cu:345-346)
        L.fc1_w = add_matrix(m, p + "ffn.fc1.weight", ffn_dim(c), D, true);
        L.fc1_b = vec(p + "ffn.fc1.bias", ffn_dim(c));
        L.fc2_w = add_matrix(m, p + "ffn.fc2.weight", D, ffn_dim(c), true);
        L.fc2_b = vec(p + "ffn.fc2.bias", D);
    }
    // final layer (dit_block.cu:392-412)
    m->fnorm = vec("final_layer.norm_final.weight", D, true);
    m->f1w = add_matrix(m, "final_layer.ffn_final.fc1.weight", D, D, false);
    m->f1b = vec("final_layer.ffn_final.fc1.bias", D);
    m->f2w = add_matrix(m, "final_layer.ffn_final.fc2.weight", c.action_dim, D, false);
    m->f2b = vec("final_layer.ffn_final.fc2.bias", c.action_dim);
}

// ---- launch helpers -------------------------------------------------------

const float* pf(sf_rdt* m, int idx) { return static_cast<const float*>(m->params[idx].data); }

// A batched K/V group's GEMM: rows x (blocks * 2D), bf16 C with the bias
// (the library path writes it directly).
sf_gemm_desc kv_group_desc(const sf_rdt* m, int g, const void* A, int rows) {
    const sf_rdt::KvGroup& G = m->kvg[g];
    const int D = m->cfg.hidden;
    sf_gemm_desc d{};
    d.M = rows;
    d.N = (int32_t)G.blocks.size() * 2 * D;
    d.K = D;
    d.A = A;
    d.lda = D;
    d.a_dtype = SF_BF16;
    d.W = G.W;
    d.ldw = D;
    d.w_dtype = G.w_dtype;
    d.w_scale = G.scale;
    d.bias = G.bias;
    d.act = SF_ACT_NONE;
    d.epilogue = SF_EPI_PLAIN;
    d.C = m->kv_prod;
    d.ldc = d.N;
    d.c_dtype = SF_BF16;
    d.workspace = m->gemm_ws;
    d.workspace_bytes = (int64_t)m->gemm_ws_bytes;
    return d;
}

// Whether group g's K/V projections run as one GEMM at this many rows: the
// library path (more than 160 rows), back-to-back weights, and a product
// that fits kv_prod.
constexpr size_t kKvProdMaxBytes = size_t(1) << 30;
bool kv_batched(const sf_rdt* m, int g, int rows) {
    const sf_rdt::KvGroup& G = m->kvg[g];
    const size_t bytes = (size_t)rows * G.blocks.size() * 2 * m->cfg.hidden * 2;
    return G.contiguous && G.blocks.size() > 1 && rows > 160 && bytes <= kKvProdMaxBytes &&
           bytes <= m->kv_prod_bytes;
}

// A as deferred-norm rows (x * gamma with m->row_ss): the output rows get
// their 1/rms after the product.
void set_row_scale(const sf_rdt* m, sf_gemm_desc& d) {
    d.a_row_ss = m->row_ss;
    d.a_row_tiles = m->cfg.hidden / 64;
    d.a_row_n = m->cfg.hidden;
    d.a_row_eps = m->cfg.eps;
}

int linear(sf_rdt* m, const void* A, int64_t lda, int M, int w_idx, int b_idx, int act, void* C,
           int64_t ldc, int c_dtype, bool accumulate, hipStream_t s, int a_dtype = SF_BF16) {
    const Param& W = m->params[w_idx];
    sf_gemm_desc d{};
    d.M = M;
    d.N = (int32_t)W.shape[0];
    d.K = (int32_t)W.shape[1];
    d.A = A;
    d.lda = lda;
    d.a_dtype = a_dtype;
    d.W = W.data;
    d.ldw = W.shape[1];
    d.w_dtype = W.dtype;
    d.w_scale = W.scale;
    d.w_codes16 = m->codes16_of[w_idx];
    d.w16_f16 = d.w_codes16 ? 1 : 0;
    d.bias = b_idx >= 0 ? pf(m, b_idx) : nullptr;
    d.act = act;
    d.epilogue = SF_EPI_PLAIN;
    d.C = C;
    d.ldc = ldc;
    d.c_dtype = c_dtype;
    d.accumulate = accumulate ? 1 : 0;
    d.workspace = m->gemm_ws;
    d.workspace_bytes = (int64_t)m->gemm_ws_bytes;
    return sf_gemm(&d, s);
}

// x += A W^T + b (fp32 residual m->x, A in a_dtype), then
// out = rmsnorm(x) * gamma in out_dtype.  At more than 160 rows the branch
// output is stored in bf16 before the add (round_product), as the
// reference's projection returns it (dit_block.cu:233, 321, 160).
int linear_add_norm(sf_rdt* m, const void* A, int a_dtype, int M, int w_idx, int b_idx, int gamma_idx,
                    void* out, int out_dtype, hipStream_t s, bool deferred = false) {
    const Param& W = m->params[w_idx];
    const int D = m->cfg.hidden;
    sf_gemm_desc d{};
    d.M = M;
    d.N = (int32_t)W.shape[0];
    d.K = (int32_t)W.shape[1];
    d.A = A;
    d.lda = W.shape[1];
    d.a_dtype = a_dtype;
    d.W = W.data;
    d.ldw = W.shape[1];
    d.w_dtype = W.dtype;
    d.w_scale = W.scale;
    d.w_codes16 = m->codes16_of[w_idx];
    d.w16_f16 = d.w_codes16 ? 1 : 0;
    d.bias = pf(m, b_idx);
    d.epilogue = SF_EPI_ADD_NORM;
    d.C = m->x;
    d.ldc = D;
    d.c_dtype = SF_F32;
    d.eps = m->cfg.eps;
    d.norm_gamma = pf(m, gamma_idx);
    d.norm_out = out;
    d.norm_ldo = D;
    d.norm_dtype = out_dtype;
    d.workspace = m->gemm_ws;
    d.workspace_bytes = (int64_t)m->gemm_ws_bytes;
    d.round_product = 1;
    if (deferred) d.norm_ss = m->row_ss;
    return sf_gemm(&d, s);
}

// Per-head projection: sections of H*64 columns -> [B, H, S, 64] bf16.
// round_product: above 160 rows the projection is stored in bf16 before the
// per-head RMSNorm, as the reference's qkv / q / kv projection output is
// (dit_block.cu:207, 284, 291).
int linear_heads(sf_rdt* m, const void* A, int M, int S, int w_idx, int b_idx,
                 uint16_t* const* outs, const int* gamma_idx, int nsec, hipStream_t s,
                 int a_dtype = SF_BF16, bool round_product = false, bool a_deferred = false) {
    const Param& W = m->params[w_idx];
    const int H = m->cfg.heads;
    sf_gemm_desc d{};
    d.M = M;
    d.N = (int32_t)W.shape[0];
    d.K = (int32_t)W.shape[1];
    d.A = A;
    d.lda = W.shape[1];
    d.a_dtype = a_dtype;
    d.W = W.data;
    d.ldw = W.shape[1];
    d.w_dtype = W.dtype;
    d.w_scale = W.scale;
    d.w_codes16 = m->codes16_of[w_idx];
    d.w16_f16 = d.w_codes16 ? 1 : 0;
    d.bias = pf(m, b_idx);
    d.epilogue = SF_EPI_HEADS;
    d.H = H;
    d.S = S;
    d.eps = m->cfg.eps;
    for (int j = 0; j < nsec; ++j) {
        d.head_out[j] = outs[j];
        d.head_gamma[j] = gamma_idx[j] >= 0 ? pf(m, gamma_idx[j]) : nullptr;
        d.head_stride[j][0] = (int64_t)H * S * 64;
        d.head_stride[j][1] = (int64_t)S * 64;
        d.head_stride[j][2] = 64;
    }
    d.workspace = m->gemm_ws;
    d.workspace_bytes = (int64_t)m->gemm_ws_bytes;
    d.round_product = round_product ? 1 : 0;
    if (a_deferred) set_row_scale(m, d);
    return sf_gemm(&d, s);
}

// Q of a cross-attention given as the cross-q projection's split-K
// partials (sf_attn_desc.q_partials); row_ss: their input rows were
// deferred-norm rows.
struct QPartials {
    const float* p = nullptr;
    int splits = 0;
    const float* bias = nullptr;
    const float* scale = nullptr;
    const float* gamma = nullptr;
    const float* row_ss = nullptr;
};

// Q (and for the self-attention K, V) read from a projection's bf16 output
// rows instead of [B, H, S, 64]: row b*S + s, row length q_ld / kv_ld
// elements, head h at column h*64; q_gamma / k_gamma: the per-head norms the
// attention applies as it loads them.
struct RowsIn {
    int64_t q_ld = 0;
    int64_t kv_ld = 0;   // 0: K, V in [B, H, Sc, 64]
    const float* q_gamma = nullptr;
    const float* k_gamma = nullptr;
    bool f16 = false;    // rows in fp16: with kv_ld, Q, K and V (an fp16 attention); else Q only
};

// Sc: the rows per head of the K/V buffer (its capacity), Sk <= Sc the keys
// read.  qp: Q from partials instead of q (which is then not read).
int attention(sf_rdt* m, const uint16_t* q, const uint16_t* k, const uint16_t* v, int Sk,
              const int32_t* valid_len, void* out, bool exact_pv, hipStream_t s, int Sc = 0,
              const QPartials* qp = nullptr, const RowsIn* rows = nullptr, bool v_f16 = false) {
    const sf_rdt_config& c = m->cfg;
    const int S = c.horizon + 3;
    sf_attn_desc d;
    const bool all16 = rows && rows->f16 && rows->kv_ld;
    sf_attn_desc_init_bhsd(&d, c.batch, c.heads, S, Sk, 64, all16 ? SF_F16 : SF_BF16, m->act16);
    if (rows && rows->f16 && !rows->kv_ld) d.q_f16 = 1;
    if (rows) {
        d.q_stride[0] = (int64_t)S * rows->q_ld;
        d.q_stride[1] = 64;
        d.q_stride[2] = rows->q_ld;
        if (rows->kv_ld) {
            for (int64_t* st : {d.k_stride, d.v_stride}) {
                st[0] = (int64_t)Sk * rows->kv_ld;
                st[1] = 64;
                st[2] = rows->kv_ld;
            }
        }
        d.q_gamma = rows->q_gamma;
        d.k_gamma = rows->k_gamma;
        d.q_eps = c.eps;
    }
    if (Sc > Sk) {
        d.k_stride[0] = d.v_stride[0] = (int64_t)c.heads * Sc * 64;
        d.k_stride[1] = d.v_stride[1] = (int64_t)Sc * 64;
        // the split count of the full buffer: its key splits are shares of
        // the valid keys, which already lie below Sk (fewer, longer splits
        // for the shorter key range measured slower: 8.9 vs 7.9 us per
        // call at batch 1)
        if (Sk > 128) {
            sf_attn_desc full = d;
            full.Sk = Sc;
            d.num_splits = sf_attn_num_splits(&full);
        }
    }
    d.kv_valid_len = valid_len;
    d.exact_pv = exact_pv ? 1 : 0;
    d.v_f16 = v_f16 ? 1 : 0;
    if (qp) {
        d.q_partials = qp->p;
        d.q_splits = qp->splits;
        d.q_bias = qp->bias;
        d.q_scale = qp->scale;
        d.q_gamma = qp->gamma;
        d.q_eps = c.eps;
        if (qp->row_ss) {
            d.q_row_ss = qp->row_ss;
            d.q_row_tiles = c.hidden / 64;
            d.q_row_n = c.hidden;
            d.q_row_eps = c.eps;
        }
    }
    // output straight into [B, S, H*64] (head_to_seq fused away)
    d.o_stride[0] = (int64_t)S * c.hidden;
    d.o_stride[1] = 64;
    d.o_stride[2] = c.hidden;
    return sf_attn_fwd(&d, q, k, v, out, m->attn_ws, m->attn_ws_bytes, s);
}

// The cross-q projection of block L over the M rows of m->n, left as its
// split-K partials in the GEMM workspace (SF_EPI_PARTIALS); *qp describes
// them for the language attention, which finishes Q (bias, int8 scale,
// q_norm) as the heads epilogue would (dit_block.cu:282-307).
int cross_q_partials(sf_rdt* m, const LayerIdx& L, int M, hipStream_t s, QPartials* qp) {
    const Param& W = m->params[L.cq_w];
    sf_gemm_desc d{};
    d.M = M;
    d.N = (int32_t)W.shape[0];
    d.K = (int32_t)W.shape[1];
    d.A = m->n;
    d.lda = m->cfg.hidden;
    d.a_dtype = SF_BF16;
    d.W = W.data;
    d.ldw = W.shape[1];
    d.w_dtype = W.dtype;
    d.w_scale = W.scale;
    d.epilogue = SF_EPI_PARTIALS;
    d.workspace = m->gemm_ws;
    d.workspace_bytes = (int64_t)m->gemm_ws_bytes;
    SF_TRY(sf_gemm(&d, s));
    qp->p = static_cast<const float*>(m->gemm_ws);
    qp->splits = m->cq_splits;
    qp->bias = pf(m, L.cq_b);
    qp->scale = W.scale;
    qp->gamma = pf(m, L.cq_norm);
    qp->row_ss = m->n_deferred ? m->row_ss : nullptr;
    return SF_OK;
}

// The projection weights that get fp16 copies.  Above 160 rows (the
// library path): every block's six and the final layer's two.  At most 160
// rows, with bf16 weights: the matrices whose inputs are fp16 there -- each
// block's fc1 and fc2 and the final layer's fc2 -- so the split-K kernel
// reads fp16 operands instead of converting every bf16 fragment in
// registers (the same operands, so the same results); int8 weights keep
// their 1-byte codes.  Only matrices with K a multiple of 16.  With
// int8_weights = 2, no copy of the int8 matrices sf_gemm multiplies directly
// at the block's rows (sf_gemm_int8_direct; every such call the block makes
// has fp16 activations and a 16-bit fp16 product).
std::vector<int> w16_params(const sf_rdt* m) {
    const sf_rdt_config& c = m->cfg;
    std::vector<int> ws;
    const int rows = c.batch * (c.horizon + 3);
    if (rows > 160) {
        for (const LayerIdx& L : m->layers)
            for (int w : block_weights(L)) ws.push_back(w);
        ws.push_back(m->f1w);
        ws.push_back(m->f2w);
        if (c.int8_weights == 2) {
            std::vector<int> keep;
            for (int w : ws) {
                const Param& P = m->params[w];
                sf_gemm_desc d{};
                d.M = rows;
                d.N = (int32_t)P.shape[0];
                d.K = (int32_t)P.shape[1];
                d.lda = d.K;
                d.a_dtype = SF_F16;
                d.ldw = P.shape[1];
                d.w_dtype = P.dtype;
                d.epilogue = SF_EPI_PLAIN;
                d.c_dtype = SF_F16;
                if (!sf_gemm_int8_direct(&d)) keep.push_back(w);
            }
            ws.swap(keep);
        }
    } else if (!c.int8_weights) {
        for (const LayerIdx& L : m->layers) {
            ws.push_back(L.fc1_w);
            ws.push_back(L.fc2_w);
        }
        ws.push_back(m->f2w);
    }
    std::vector<int> out;
    for (int w : ws)
        if (m->params[w].shape[1] % 16 == 0) out.push_back(w);
    return out;
}

// Every GEMM the runtime issues: each matrix at each row count it is used
// with (step rows B*S, B*T, B, 1; condition rows B*lang_max, B*img_len).
// Returns the largest workspace; with prepare, also selects the library
// path's algorithms now, outside any graph capture.
size_t gemm_ws_for(const sf_rdt* m, bool prepare, int* status) {
    const sf_rdt_config& c = m->cfg;
    const int rows[7] = {c.batch * (c.horizon + 3), c.batch * c.horizon, c.batch, 1,
                         c.batch * c.lang_max, c.batch * c.img_len,
                         std::min(160, c.lang_max)};   // largest split-K M (language rows at batch 1)
    size_t best = 0;
    // weights with an fp16 copy (above 160 rows) multiply fp16 activations
    // in fp16 on the library path
    std::vector<char> w16(m->params.size(), 0);
    if (c.batch * (c.horizon + 3) > 160)
        for (int w : w16_params(m)) w16[w] = 1;
    for (size_t pi = 0; pi < m->params.size(); ++pi) {
        const Param& p = m->params[pi];
        if (p.shape.size() != 2 || p.dtype == SF_F32) continue;
        for (int M : rows) {
            for (int ad : {SF_BF16, SF_F16}) {
                sf_gemm_desc d{};
                d.M = M;
                d.N = (int32_t)p.shape[0];
                d.K = (int32_t)p.shape[1];
                d.lda = d.K;
                d.a_dtype = ad;
                d.ldw = d.K;
                d.w_dtype = p.dtype;
                d.w16_f16 = ad == SF_F16 && w16[pi];
                best = std::max(best, sf_gemm_workspace_bytes(&d));
                if (prepare && status && *status == SF_OK) *status = sf_gemm_prepare(&d);
            }
        }
    }
    // each condition group's K/V projections as one GEMM (kv_batched)
    for (int g = 0; g < 2; ++g) {
        const int rows = m->kvg[g].rows_max;
        if (!kv_batched(m, g, rows)) continue;
        sf_gemm_desc d = kv_group_desc(m, g, nullptr, rows);
        best = std::max(best, sf_gemm_workspace_bytes(&d));
        if (g == 0 && c.batch == 1) d.M = m->lang_rows;   // the language rows set now
        if (prepare && status && *status == SF_OK && kv_batched(m, g, d.M)) *status = sf_gemm_prepare(&d);
    }
    return best;
}

size_t attn_ws_for(const sf_rdt_config& c, int Sk) {
    sf_attn_desc d;
    sf_attn_desc_init_bhsd(&d, c.batch, c.heads, c.horizon + 3, Sk, 64, SF_BF16, SF_BF16);
    return sf_attn_workspace_bytes(&d);
}

// TimestepEmbedding::forward (dit_block.cu:102-127): sincos row -> Linear +
// SiLU -> Linear, fp32 [D] out.
int timestep_embed(sf_rdt* m, const int* idx4, int step, float* out, hipStream_t s) {
    const sf_rdt_config& c = m->cfg;
    if (step < 0) step = 0;
    if (step > c.num_train_timesteps - 1) step = c.num_train_timesteps - 1;
    const uint16_t* row = m->sincos + (int64_t)step * c.freq_dim;
    SF_TRY(linear(m, row, c.freq_dim, 1, idx4[0], idx4[1], SF_ACT_SILU, m->emb_h, c.hidden, SF_BF16,
                  false, s));
    return linear(m, m->emb_h, c.hidden, 1, idx4[2], idx4[3], SF_ACT_NONE, out, c.hidden, SF_F32,
                  false, s);
}

// Gamma of the RMSNorm that follows block i: the next block's norm1, or the
// final layer's norm after the last block.
int next_norm(const sf_rdt* m, int i) {
    return i + 1 < m->cfg.layers ? m->layers[i + 1].norm1 : m->fnorm;
}

// Refreshes the fp16 weight copies of blocks [first, first + count) and,
// with final_layer, of the final layer (no-op without copies), up to
// SF_CODES_MAX_JOBS matrices per launch.
int widen_codes(sf_rdt* m, int first, int count, hipStream_t s, bool final_layer = false) {
    if (!m->codes16) return SF_OK;
    sf_w16_job jobs[SF_CODES_MAX_JOBS];
    int n = 0;
    std::vector<int> ws;
    for (int i = first; i < first + count; ++i)
        for (int w : block_weights(m->layers[i])) ws.push_back(w);
    if (final_layer) {
        ws.push_back(m->f1w);
        ws.push_back(m->f2w);
    }
    for (int w : ws) {
        const Param& P = m->params[w];
        if (!m->codes16_of[w]) continue;
        jobs[n].w = P.data;
        jobs[n].w_dtype = P.dtype;
        jobs[n].ldw = P.shape[1];
        jobs[n].out = const_cast<void*>(m->codes16_of[w]);
        jobs[n].N = (int32_t)P.shape[0];
        jobs[n].K = (int32_t)P.shape[1];
        if (++n == SF_CODES_MAX_JOBS) {
            SF_TRY(sf_weights_to_f16(jobs, n, s));
            n = 0;
        }
    }
    return n ? sf_weights_to_f16(jobs, n, s) : SF_OK;
}

// RDTBlock::forward (dit_block.cu:349-387) on the fp32 residual m->x, with
// m->n holding norm1(x) on entry; on exit m->n holds the next norm of x.
// The fp16 weight copies of the library path (if any) are current
// (refresh_w16).
int block_forward(sf_rdt* m, int i, hipStream_t s) {
    const sf_rdt_config& c = m->cfg;
    const LayerIdx& L = m->layers[i];
    const int D = c.hidden, S = c.horizon + 3, M = c.batch * S;
    const int fd = m->ffn_dtype, ad = m->act16;
    // self-attention branch
    if (m->rows_qkv) {
        // qkv = x W^T + b in fp16 (dit_block.cu:206-207); split_qkv and
        // apply_qk_norm (:209-220) happen as the attention loads the rows
        SF_TRY(linear(m, m->n, D, M, L.qkv_w, L.qkv_b, SF_ACT_NONE, m->qkv_rows, 3 * D, ad, false, s, ad));
        RowsIn r;
        r.q_ld = r.kv_ld = 3 * D;
        r.q_gamma = pf(m, L.q_norm);
        r.k_gamma = pf(m, L.k_norm);
        r.f16 = ad == SF_F16;
        SF_TRY(attention(m, m->qkv_rows, m->qkv_rows + D, m->qkv_rows + 2 * D, S, nullptr, m->a, false, s, 0,
                         nullptr, &r));
    } else {
        uint16_t* qkv[3] = {m->q, m->k, m->v};
        const int qk_g[3] = {L.q_norm, L.k_norm, -1};
        SF_TRY(linear_heads(m, m->n, M, S, L.qkv_w, L.qkv_b, qkv, qk_g, 3, s, SF_BF16, true, m->n_deferred));
        SF_TRY(attention(m, m->q, m->k, m->v, S, nullptr, m->a, false, s));
    }
    SF_TRY(linear_add_norm(m, m->a, ad, M, L.proj_w, L.proj_b, L.norm2, m->n, ad, s, m->defer));
    m->n_deferred = m->defer;
    // cross-attention branch: even blocks attend to language, odd to image
    // (dit_block.cu:369)
    const bool lang = (i % 2) == 0;
    // the cached V of a layer on the fp16 P.V form is held in fp16 (converted
    // once when the condition was set, sf_bf16_to_f16_below)
    const bool exact = m->exact_pv[i] != 0;
    if (lang && m->cq_splits > 0) {   // Q finished inside the attention
        QPartials qp;
        SF_TRY(cross_q_partials(m, L, M, s, &qp));
        SF_TRY(attention(m, nullptr, m->ck[i], m->cv[i], m->cond_lang_rows, m->lang_len, m->a,
                         exact, s, c.lang_max, &qp, nullptr, !exact));
    } else if (m->rows_qkv) {
        // q = x W^T + b in fp16 rows (dit_block.cu:282-284); seq_to_head and
        // q_norm (:298-307) happen as the attention loads them (rounding Q to
        // bf16 for the bf16 K/V cache)
        SF_TRY(linear(m, m->n, D, M, L.cq_w, L.cq_b, SF_ACT_NONE, m->q, D, ad, false, s, ad));
        RowsIn r;
        r.q_ld = D;
        r.q_gamma = pf(m, L.cq_norm);
        r.f16 = ad == SF_F16;
        SF_TRY(attention(m, m->q, m->ck[i], m->cv[i], lang ? m->cond_lang_rows : c.img_len,
                         lang ? m->lang_len : nullptr, m->a, exact, s,
                         lang ? c.lang_max : c.img_len, nullptr, &r, !exact));
    } else {
        uint16_t* cq[1] = {m->q};
        const int cq_g[1] = {L.cq_norm};
        SF_TRY(linear_heads(m, m->n, M, S, L.cq_w, L.cq_b, cq, cq_g, 1, s, SF_BF16, true, m->n_deferred));
        SF_TRY(attention(m, m->q, m->ck[i], m->cv[i], lang ? m->cond_lang_rows : c.img_len,
                         lang ? m->lang_len : nullptr, m->a, exact, s,
                         lang ? c.lang_max : c.img_len, nullptr, nullptr, !exact));
    }
    SF_TRY(linear_add_norm(m, m->a, ad, M, L.cproj_w, L.cproj_b, L.norm3, m->n3, fd, s));
    // FFN branch (Mlp::forward, dit_block.cu:143-163); fc2's add + norm
    // writes the next block's norm1 (act16, the QKV input)
    const int F = (int)ffn_dim(c);
    SF_TRY(linear(m, m->n3, D, M, L.fc1_w, L.fc1_b, SF_ACT_GELU_TANH, m->h, F, fd, false, s, fd));
    // the next block's norm1 deferred; the final norm row-wide (its consumer,
    // the final layer's fc1, takes normalised rows)
    const bool defer_next = m->defer && i + 1 < c.layers;
    SF_TRY(linear_add_norm(m, m->h, fd, M, L.fc2_w, L.fc2_b, next_norm(m, i), m->n, ad, s, defer_next));
    m->n_deferred = defer_next;
    return SF_OK;
}

// m->n = first norm applied to the residual m->x before block `first`.
int entry_norm(sf_rdt* m, int first, hipStream_t s) {
    const sf_rdt_config& c = m->cfg;
    const int D = c.hidden, M = c.batch * (c.horizon + 3);
    const int g = first < c.layers ? m->layers[first].norm1 : m->fnorm;
    m->n_deferred = m->defer && first < c.layers;
    if (m->n_deferred) return sf_rmsnorm_deferred(m->x, D, pf(m, g), m->n, m->act16, D, m->row_ss, M, D, s);
    return sf_rmsnorm(m->x, SF_F32, D, pf(m, g), m->n, m->act16, D, M, D, c.eps, s);
}

// The timestep index of t (rdt1b.cpp:312-313): round(t * (T_train - 1)).
int timestep_index(const sf_rdt_config& c, float t) {
    const float tt = t * (float)(c.num_train_timesteps - 1);
    return (int)std::lround(tt);
}

// RDT1BModel::denoise_step up to the final layer: velocity rows [B*S, A].
// t_emb_given: t's timestep token already embedded (the sampler's schedule),
// else it is embedded here.
int step_forward(sf_rdt* m, const float* x_t, float t, hipStream_t s,
                 const float* t_emb_given = nullptr) {
    const sf_rdt_config& c = m->cfg;
    const int D = c.hidden, T = c.horizon, A = c.action_dim, S = T + 3;
    const int BT = c.batch * T, M = c.batch * S;
    // action tokens: state_adaptor(cat(x_t, ones)) (rdt1b.cpp:286-302)
    SF_TRY(sf_build_action_input(x_t, m->act_in, BT, A, s));
    SF_TRY(linear(m, m->act_in, 2 * A, BT, m->sa[0], m->sa[1], SF_ACT_GELU_TANH, m->sa0, D, SF_BF16,
                  false, s));
    SF_TRY(linear(m, m->sa0, D, BT, m->sa[2], m->sa[3], SF_ACT_GELU_TANH, m->sa1, D, SF_BF16, false,
                  s));
    SF_TRY(linear(m, m->sa1, D, BT, m->sa[4], m->sa[5], SF_ACT_NONE, m->act_out, D, SF_F32, false, s));
    // timestep token (rdt1b.cpp:312-315); the frequency token is cached
    const float* t_emb = t_emb_given;
    if (!t_emb) {
        SF_TRY(timestep_embed(m, m->te, timestep_index(c, t), m->t_emb, s));
        t_emb = m->t_emb;
    }
    SF_TRY(sf_assemble_tokens(m->x, t_emb, m->f_emb, m->state_tok, m->act_out, pf(m, m->xpos),
                              c.batch, T, D, s));
    SF_TRY(entry_norm(m, 0, s));
    for (int i = 0; i < c.layers; ++i) SF_TRY(block_forward(m, i, s));
    // FinalLayer (dit_block.cu:407-412); m->n = norm_final(x) from the last block
    SF_TRY(linear(m, m->n, D, M, m->f1w, m->f1b, SF_ACT_GELU_TANH, m->h, D, m->ffn_dtype, false, s, m->act16));
    return linear(m, m->h, D, M, m->f2w, m->f2b, SF_ACT_NONE, m->vel_rows, A, SF_F32, false, s,
                  m->ffn_dtype);
}

std::vector<float> schedule(int num_steps) {
    // Schedule::linspace (flow_matching.cpp:10-17), float arithmetic
    std::vector<float> ts(num_steps + 1);
    for (int i = 0; i <= num_steps; ++i) {
        const float alpha = (float)i / (float)num_steps;
        ts[i] = 1.f + alpha * (0.f - 1.f);
    }
    return ts;
}

int sample_body(sf_rdt* m, hipStream_t s) {
    const sf_rdt_config& c = m->cfg;
    const std::vector<float> ts = schedule(c.num_steps);
    for (int step = 0; step < c.num_steps; ++step) {
        SF_TRY(step_forward(m, m->x_state, ts[step], s, m->t_emb_steps + (size_t)step * c.hidden));
        const float dt = ts[step + 1] - ts[step];
        SF_TRY(sf_euler_update(m->x_state, m->vel_rows, c.batch, c.horizon, c.action_dim,
                               c.horizon + 3, dt, s));
    }
    return SF_OK;
}

void release_graph(sf_rdt* m) {
    if (m->graph_exec) (void)hipGraphExecDestroy(m->graph_exec);
    if (m->graph) (void)hipGraphDestroy(m->graph);
    m->graph_exec = nullptr;
    m->graph = nullptr;
    m->graph_stream = nullptr;
}

// Chooses each layer's P.V form for the condition set last (waits for its
// max |V| once per condition; never under capture).  A change of forms
// invalidates the captured loop.
int resolve_pv_forms(sf_rdt* m) {
    if (m->forms_gen == m->cond_gen) return SF_OK;
    SF_HIP(hipEventSynchronize(m->cond_event));
    bool changed = false;
    for (int i = 0; i < m->cfg.layers; ++i) {
        const uint8_t exact = m->v_absmax_host[i] < 65504.f ? 0 : 1;   // NaN compares false
        changed |= exact != m->exact_pv[i];
        m->exact_pv[i] = exact;
    }
    if (changed) release_graph(m);
    m->forms_gen = m->cond_gen;
    return SF_OK;
}

hipStream_t pick_stream(sf_rdt* m, void* stream) {
    return stream ? static_cast<hipStream_t>(stream) : m->own_stream;
}

// The fp16 weight copies of the library path, brought up to date before a
// pass (never under capture: every entry point calls this first).
int refresh_w16(sf_rdt* m, hipStream_t s) {
    if (!m->codes16 || !m->w16_stale) return SF_OK;
    SF_TRY(widen_codes(m, 0, m->cfg.layers, s, true));
    m->w16_stale = false;
    return SF_OK;
}

}  // namespace

extern "C" void sf_rdt_config_default(sf_rdt_config* c) {
    if (!c) return;
    *c = sf_rdt_config{};
    c->hidden = 2048;
    c->layers = 28;
    c->heads = 32;
    c->action_dim = 128;
    c->horizon = 64;
    c->freq_dim = 256;
    c->state_dim = 128;
    c->lang_max = 1024;
    c->img_len = 4374;
    c->lang_token_dim = 4096;
    c->img_token_dim = 1152;
    c->num_train_timesteps = 1000;
    c->ctrl_freq = 25;
    c->num_steps = 5;
    c->batch = 1;
    c->int8_weights = 0;
    c->eps = 1e-6f;
    c->mlp_ratio = 1;
}

extern "C" int sf_rdt_create(const sf_rdt_config* cfg, sf_rdt** out) {
    if (!cfg || !out) return SF_EINVAL;
    *out = nullptr;
    const sf_rdt_config& c = *cfg;
    if (c.hidden <= 0 || c.heads <= 0 || c.hidden != c.heads * 64) return SF_ENOTSUP;
    if (c.layers < 0 || c.batch <= 0 || c.horizon <= 0 || c.action_dim <= 0 || c.num_steps <= 0)
        return SF_EINVAL;
    if (c.mlp_ratio < 0 || c.mlp_ratio > 8) return SF_EINVAL;
    if (c.lang_max <= 0 || c.img_len <= 0 || c.freq_dim <= 0 || c.num_train_timesteps <= 0)
        return SF_EINVAL;
    if ((c.hidden | c.freq_dim | c.lang_token_dim | c.img_token_dim | (2 * c.state_dim) |
         (2 * c.action_dim)) & 31)
        return SF_ENOTSUP;   // GEMM K dims are multiples of 32
    sf_rdt* m = new sf_rdt();
    m->cfg = c;
    // fp16 FFN inputs at every batch size; the other projection inputs in
    // fp16 once the block GEMMs leave the split-K regime (M > 160 rows)
    m->ffn_dtype = SF_F16;
    m->act16 = c.batch * (c.horizon + 3) <= 160 ? SF_BF16 : SF_F16;
    m->defer = c.batch * (c.horizon + 3) <= 160 && c.hidden % 64 == 0 && c.hidden / 64 <= 64;
    build_param_table(m);

    const int64_t B = c.batch, D = c.hidden, T = c.horizon, S = T + 3, A = c.action_dim;
    const int64_t H = c.heads;
    // arena layout: parameters (each condition group's K/V projections back
    // to back), then buffers
    size_t off = 0;
    std::vector<char> in_group(m->params.size(), 0);
    for (int i = 0; i < c.layers; ++i) {
        m->kvg[i % 2].blocks.push_back(i);
        in_group[m->layers[i].ckv_w] = in_group[m->layers[i].ckv_b] = 1;
    }
    for (size_t j = 0; j < m->params.size(); ++j) {
        if (in_group[j]) continue;
        Param& p = m->params[j];
        p.offset = off;
        off += align256(p.bytes());
        if (p.dtype == SF_I8) {
            p.scale_offset = off;
            off += align256((size_t)p.shape[0] * 4);
        }
    }
    size_t kv_w_off[2] = {0, 0}, kv_b_off[2] = {0, 0}, kv_s_off[2] = {0, 0};
    for (int g = 0; g < 2; ++g) {
        sf_rdt::KvGroup& G = m->kvg[g];
        if (G.blocks.empty()) continue;
        const Param& W0 = m->params[m->layers[G.blocks[0]].ckv_w];
        const Param& B0 = m->params[m->layers[G.blocks[0]].ckv_b];
        G.w_dtype = W0.dtype;
        // back to back when every piece is a multiple of 256 bytes (always
        // for D = 64 * heads); otherwise the group runs per block
        G.contiguous = W0.bytes() % 256 == 0 && B0.bytes() % 256 == 0 && (W0.shape[0] * 4) % 256 == 0;
        kv_w_off[g] = off;
        for (int i : G.blocks) {
            m->params[m->layers[i].ckv_w].offset = off;
            off += align256(m->params[m->layers[i].ckv_w].bytes());
        }
        kv_b_off[g] = off;
        for (int i : G.blocks) {
            m->params[m->layers[i].ckv_b].offset = off;
            off += align256(m->params[m->layers[i].ckv_b].bytes());
        }
        kv_s_off[g] = off;
        for (int i : G.blocks) {
            Param& p = m->params[m->layers[i].ckv_w];
            if (p.dtype != SF_I8) continue;
            p.scale_offset = off;
            off += align256((size_t)p.shape[0] * 4);
        }
        G.rows_max = g == 0 ? (int)(B * c.lang_max) : (int)(B * c.img_len);
        const size_t prod = (size_t)G.rows_max * G.blocks.size() * 2 * D * 2;
        if (G.contiguous && G.blocks.size() > 1 && G.rows_max > 160 && prod <= kKvProdMaxBytes)
            m->kv_prod_bytes = std::max(m->kv_prod_bytes, prod);
    }
    struct Buf { void** ptr; size_t bytes; };
    const int64_t adapt_rows = B * std::max(c.lang_max, c.img_len);
    m->ck.assign(c.layers, nullptr);
    m->cv.assign(c.layers, nullptr);
    std::vector<Buf> bufs = {
        {(void**)&m->x, (size_t)(B * S * D * 4)},
        {(void**)&m->n, (size_t)(B * S * D * 2)},
        {(void**)&m->q, (size_t)(B * H * S * 64 * 2)},
        {(void**)&m->k, (size_t)(B * H * S * 64 * 2)},
        {(void**)&m->v, (size_t)(B * H * S * 64 * 2)},
        {(void**)&m->a, (size_t)(B * S * D * 2)},
        {(void**)&m->n3, (size_t)(B * S * D * 2)},
        {(void**)&m->h, (size_t)(B * S * ffn_dim(c) * 2)},
        {(void**)&m->act_in, (size_t)(B * T * 2 * A * 2)},
        {(void**)&m->sa0, (size_t)(B * T * D * 2)},
        {(void**)&m->sa1, (size_t)(B * T * D * 2)},
        {(void**)&m->act_out, (size_t)(B * T * D * 4)},
        {(void**)&m->sincos, (size_t)c.num_train_timesteps * c.freq_dim * 2},
        {(void**)&m->emb_h, (size_t)(D * 2)},
        {(void**)&m->t_emb, (size_t)(D * 4)},
        {(void**)&m->f_emb, (size_t)(D * 4)},
        {(void**)&m->t_emb_steps, (size_t)c.num_steps * D * 4},
        {(void**)&m->state_tok, (size_t)(B * D * 2)},
        {(void**)&m->vel_rows, (size_t)(B * S * A * 4)},
        {(void**)&m->x_state, (size_t)(B * T * A * 4)},
        {(void**)&m->x_infer, (size_t)(B * T * A * 4)},
        {(void**)&m->lang_len, (size_t)(B * 4)},
        {(void**)&m->v_absmax, (size_t)std::max(c.layers, 1) * 4},
        {(void**)&m->lang_c, (size_t)(B * c.lang_max * D * 2)},
        {(void**)&m->img_c, (size_t)(B * c.img_len * D * 2)},
        {(void**)&m->ad_h, (size_t)(adapt_rows * D * 2)},
    };
    for (int i = 0; i < c.layers; ++i) {
        const int64_t Sc = (i % 2 == 0) ? c.lang_max : c.img_len;
        bufs.push_back({(void**)&m->ck[i], (size_t)(B * H * Sc * 64 * 2)});
        bufs.push_back({(void**)&m->cv[i], (size_t)(B * H * Sc * 64 * 2)});
    }
    m->attn_ws_bytes = std::max(attn_ws_for(c, c.lang_max), attn_ws_for(c, c.img_len));
    m->attn_ws_bytes = std::max(m->attn_ws_bytes, attn_ws_for(c, (int)S));
    bufs.push_back({&m->attn_ws, std::max<size_t>(m->attn_ws_bytes, 256)});
    if (m->kv_prod_bytes) bufs.push_back({(void**)&m->kv_prod, m->kv_prod_bytes});
    m->gemm_ws_bytes = gemm_ws_for(m, false, nullptr);
    bufs.push_back({&m->gemm_ws, std::max<size_t>(m->gemm_ws_bytes, 256)});
    m->rows_qkv = S * B > 160;
    if (m->rows_qkv) bufs.push_back({(void**)&m->qkv_rows, (size_t)(B * S * 3 * D * 2)});
    if (m->defer) bufs.push_back({(void**)&m->row_ss, (size_t)(D / 64) * B * S * 4});
    for (int w : w16_params(m))   // fp16 weight copies
        m->codes16_bytes += align256((size_t)m->params[w].shape[0] * m->params[w].shape[1] * 2);
    if (m->codes16_bytes) bufs.push_back({(void**)&m->codes16, m->codes16_bytes});
    std::vector<size_t> boff(bufs.size());
    for (size_t i = 0; i < bufs.size(); ++i) {
        boff[i] = off;
        off += align256(bufs[i].bytes);
    }
    m->arena_bytes = off;
    if (hipMalloc((void**)&m->arena, off) != hipSuccess) {
        delete m;
        return SF_EDEVICE;
    }
    for (Param& p : m->params) {
        p.data = m->arena + p.offset;
        if (p.dtype == SF_I8) p.scale = reinterpret_cast<float*>(m->arena + p.scale_offset);
    }
    for (int g = 0; g < 2; ++g) {
        sf_rdt::KvGroup& G = m->kvg[g];
        if (G.blocks.empty()) continue;
        G.W = m->arena + kv_w_off[g];
        G.bias = reinterpret_cast<const float*>(m->arena + kv_b_off[g]);
        G.scale = G.w_dtype == SF_I8 ? reinterpret_cast<const float*>(m->arena + kv_s_off[g]) : nullptr;
    }
    for (size_t i = 0; i < bufs.size(); ++i) *bufs[i].ptr = m->arena + boff[i];
    m->codes16_of.assign(m->params.size(), nullptr);
    if (m->codes16) {
        char* dst = m->codes16;
        for (int w : w16_params(m)) {
            const Param& P = m->params[w];
            m->codes16_of[w] = dst;
            dst += align256((size_t)P.shape[0] * P.shape[1] * 2);
        }
    }
    m->exact_pv.assign(c.layers, 0);
    m->lang_rows = m->cond_lang_rows = c.lang_max;
    if (c.layers > 0) {   // the fused cross-q finish (see cq_splits)
        sf_gemm_desc g{};
        g.M = (int32_t)(B * S);
        g.N = (int32_t)D;
        g.K = (int32_t)D;
        g.a_dtype = SF_BF16;
        const int splits = sf_gemm_num_splits(&g);
        sf_attn_desc a;
        sf_attn_desc_init_bhsd(&a, (int32_t)B, (int32_t)H, (int32_t)S, c.lang_max, 64, SF_BF16, SF_BF16);
        const bool qblocks = B * H * ((S + 79) / 80) < 256 && c.lang_max <= 1024 && sf_attn_num_splits(&a) == 1;
        if (splits >= 1 && splits <= 8 && qblocks && (size_t)splits * B * S * D * 4 <= m->gemm_ws_bytes)
            m->cq_splits = splits;
    }
    if (hipStreamCreate(&m->own_stream) != hipSuccess) {
        (void)hipFree(m->arena);
        delete m;
        return SF_EDEVICE;
    }
    if (hipEventCreateWithFlags(&m->cond_event, hipEventDisableTiming) != hipSuccess ||
        hipHostMalloc((void**)&m->v_absmax_host, (size_t)std::max(c.layers, 1) * 4) != hipSuccess) {
        sf_rdt_destroy(m);
        return SF_EDEVICE;
    }
    // sincos table, built in float as TimestepEmbedding::build_sincos_table
    // (dit_block.cu:58-72), stored bf16 (the MLP's input dtype)
    std::vector<uint16_t> tab((size_t)c.num_train_timesteps * c.freq_dim);
    const int half = c.freq_dim / 2;
    for (int step = 0; step < c.num_train_timesteps; ++step) {
        const float t = (float)step;
        for (int i = 0; i < half; ++i) {
            const float freq = std::exp(-std::log(10000.f) * (float)i / (float)half);
            const float angle = t * freq;
            const float cv_ = std::cos(angle), sv = std::sin(angle);
            auto bf = [](float f) {
                uint32_t u;
                std::memcpy(&u, &f, 4);
                u += 0x7fffu + ((u >> 16) & 1u);
                return (uint16_t)(u >> 16);
            };
            tab[(size_t)step * c.freq_dim + i] = bf(cv_);
            tab[(size_t)step * c.freq_dim + half + i] = bf(sv);
        }
    }
    // language K/V caches zeroed once: at batch 1 a condition projects only
    // its L rows, and the V range check reads whole caches
    for (int i = 0; i < c.layers; i += 2) {
        const size_t cb = (size_t)(B * H * c.lang_max * 64 * 2);
        if (hipMemset(m->ck[i], 0, cb) != hipSuccess || hipMemset(m->cv[i], 0, cb) != hipSuccess) {
            sf_rdt_destroy(m);
            return SF_EDEVICE;
        }
    }
    if (hipMemcpy(m->sincos, tab.data(), tab.size() * 2, hipMemcpyHostToDevice) != hipSuccess) {
        sf_rdt_destroy(m);
        return SF_EDEVICE;
    }
    int prep = SF_OK;
    (void)gemm_ws_for(m, true, &prep);
    if (prep != SF_OK) {
        sf_rdt_destroy(m);
        return prep;
    }
    *out = m;
    return SF_OK;
}

extern "C" void sf_rdt_destroy(sf_rdt* m) {
    if (!m) return;
    release_graph(m);
    if (m->cond_event) (void)hipEventDestroy(m->cond_event);
    if (m->v_absmax_host) (void)hipHostFree(m->v_absmax_host);
    if (m->own_stream) (void)hipStreamDestroy(m->own_stream);
    if (m->arena) (void)hipFree(m->arena);
    delete m;
}

extern "C" int sf_rdt_init_random(sf_rdt* m, uint64_t seed, float std, void* stream) {
    if (!m) return SF_EINVAL;
    hipStream_t s = pick_stream(m, stream);
    for (size_t i = 0; i < m->params.size(); ++i) {
        Param& p = m->params[i];
        const uint64_t ps = seed * 0x100000001B3ull + 0x9E37ull * (i + 1);
        if (p.ones) {
            SF_TRY(sf_fill_f32(static_cast<float*>(p.data), p.numel(), 1.f, s));
        } else if (p.dtype == SF_I8) {
            SF_TRY(sf_init_int8_rows(static_cast<int8_t*>(p.data), p.scale, p.shape[0], p.shape[1],
                                     ps, std, s));
        } else {
            SF_TRY(sf_init_normal(p.data, p.dtype, p.numel(), ps, std, s));
        }
    }
    release_graph(m);   // weights changed: a captured graph stays valid, but be explicit
    sf_rdt_weights_changed(m);
    return SF_OK;
}

extern "C" int32_t sf_rdt_num_params(const sf_rdt* m) { return m ? (int32_t)m->params.size() : 0; }

extern "C" int sf_rdt_param_info(const sf_rdt* m, int32_t idx, const char** name, int32_t* dtype,
                                 int32_t* ndim, int64_t shape[4]) {
    if (!m || idx < 0 || idx >= (int32_t)m->params.size()) return SF_EINVAL;
    const Param& p = m->params[idx];
    if (name) *name = p.name.c_str();
    if (dtype) *dtype = p.dtype;
    if (ndim) *ndim = (int32_t)p.shape.size();
    if (shape)
        for (size_t i = 0; i < 4; ++i) shape[i] = i < p.shape.size() ? p.shape[i] : 1;
    return SF_OK;
}

extern "C" void* sf_rdt_param_data(sf_rdt* m, int32_t idx) {
    if (!m || idx < 0 || idx >= (int32_t)m->params.size()) return nullptr;
    m->w16_stale = true;   // the caller may write through it before the next pass
    return m->params[idx].data;
}

extern "C" int sf_rdt_params_changed(sf_rdt* m) {
    if (!m) return SF_EINVAL;
    sf_rdt_weights_changed(m);
    return SF_OK;
}

extern "C" float* sf_rdt_param_scale(sf_rdt* m, int32_t idx) {
    if (!m || idx < 0 || idx >= (int32_t)m->params.size()) return nullptr;
    return m->params[idx].scale;
}

extern "C" int32_t sf_rdt_find_param(const sf_rdt* m, const char* name) {
    if (!m || !name) return -1;
    for (size_t i = 0; i < m->params.size(); ++i)
        if (m->params[i].name == name) return (int32_t)i;
    return -1;
}

extern "C" void* sf_rdt_cache_ptr(sf_rdt* m, int32_t layer, int32_t which_v) {
    if (!m || layer < 0 || layer >= m->cfg.layers) return nullptr;
    return which_v ? m->cv[layer] : m->ck[layer];
}

extern "C" int sf_rdt_set_condition(sf_rdt* m, const void* lang_c, const int32_t* lang_len,
                                    const void* img_c, const void* state_tok, void* stream) {
    if (!m || !lang_c || !lang_len || !img_c || !state_tok) return SF_EINVAL;
    m->infer_cond_valid = false;   // sf_rdt_infer re-encodes after a condition set here
    const sf_rdt_config& c = m->cfg;
    hipStream_t s = pick_stream(m, stream);
    const int D = c.hidden, B = c.batch;
    if (lang_len != m->lang_len)
        SF_HIP(hipMemcpyAsync(m->lang_len, lang_len, B * 4, hipMemcpyDeviceToDevice, s));
    if (state_tok != m->state_tok)
        SF_HIP(hipMemcpyAsync(m->state_tok, state_tok, (size_t)B * D * 2, hipMemcpyDeviceToDevice, s));
    // language rows: the caller's L at batch 1 (the reference's language
    // tensor is [B, L, D]); all lang_max rows of the padded layout otherwise
    if (m->cond_lang_rows != m->lang_rows) release_graph(m);   // its attention reads cond_lang_rows keys
    m->cond_lang_rows = m->lang_rows;
    const int Lr = B == 1 ? m->lang_rows : c.lang_max;
    // lang_c + lang_cond_pos_embed[:L], img_c + img_cond_pos_embed (rdt1b.cpp:342-349)
    SF_TRY(sf_add_pos_bf16(lang_c, pf(m, m->lpos), m->lang_c, B, Lr, D, s));
    SF_TRY(sf_add_pos_bf16(img_c, pf(m, m->ipos), m->img_c, B, c.img_len, D, s));
    // every block's K/V projection with k_norm, once per inference: above
    // 160 rows the projection is stored in bf16 before split_kv / k_norm, as
    // the reference's kv = gemm_bias_act(...) is (dit_block.cu:291-308) --
    // there the blocks attending to one condition run as one GEMM when it
    // fits (kv_batched), split per block by sf_heads_bf16
    for (int grp = 0; grp < 2; ++grp) {
        const sf_rdt::KvGroup& G = m->kvg[grp];
        const bool lang = grp == 0;
        const int Sc = lang ? c.lang_max : c.img_len;
        const int rows = lang && B == 1 ? Lr : B * Sc;   // batch 1: the L language rows only
        const void* A = lang ? m->lang_c : m->img_c;
        const bool batched = kv_batched(m, grp, rows);
        if (batched) {
            const sf_gemm_desc d = kv_group_desc(m, grp, A, rows);
            SF_TRY(sf_gemm(&d, s));
        }
        for (size_t j = 0; j < G.blocks.size(); ++j) {
            const int i = G.blocks[j];
            uint16_t* kv[2] = {m->ck[i], m->cv[i]};
            const int g[2] = {m->layers[i].ck_norm, -1};
            if (!batched) {
                SF_TRY(linear_heads(m, A, rows, Sc, m->layers[i].ckv_w, m->layers[i].ckv_b, kv, g, 2, s,
                                    SF_BF16, true));
                continue;
            }
            sf_gemm_desc h{};
            h.M = rows;
            h.N = 2 * D;
            h.epilogue = SF_EPI_HEADS;
            h.H = c.heads;
            h.S = Sc;
            h.eps = c.eps;
            for (int q = 0; q < 2; ++q) {
                h.head_out[q] = kv[q];
                h.head_gamma[q] = g[q] >= 0 ? pf(m, g[q]) : nullptr;
                h.head_stride[q][0] = (int64_t)c.heads * Sc * 64;
                h.head_stride[q][1] = (int64_t)Sc * 64;
                h.head_stride[q][2] = 64;
            }
            const int64_t ldp = (int64_t)G.blocks.size() * 2 * D;
            SF_TRY(sf_heads_bf16(&h, m->kv_prod + j * 2 * D, ldp, s));
        }
    }
    // each layer's max |V| for the choice of P.V form (resolve_pv_forms)
    if (c.layers > 0) {
        SF_TRY(sf_fill_f32(m->v_absmax, c.layers, 0.f, s));
        for (int i0 = 0; i0 < c.layers; i0 += SF_ABSMAX_MAX_JOBS) {
            sf_absmax_job jobs[SF_ABSMAX_MAX_JOBS];
            const int n = std::min(SF_ABSMAX_MAX_JOBS, c.layers - i0);
            for (int j = 0; j < n; ++j) {
                const int i = i0 + j;
                const int64_t Sc = (i % 2 == 0) ? c.lang_max : c.img_len;
                jobs[j] = sf_absmax_job{m->cv[i], (int64_t)B * c.heads * Sc * 64, m->v_absmax + i};
            }
            SF_TRY(sf_absmax_bf16_batched(jobs, n, s));
            // V of every layer below the fp16 range limit -- the layers
            // resolve_pv_forms puts on the fp16 P.V form, by the same
            // comparison -- to fp16 in place, the rounding the attention
            // would otherwise apply to every tile of every step
            SF_TRY(sf_bf16_to_f16_below(jobs, n, 65504.f, s));
        }
        SF_HIP(hipMemcpyAsync(m->v_absmax_host, m->v_absmax, (size_t)c.layers * 4, hipMemcpyDeviceToHost, s));
        SF_HIP(hipEventRecord(m->cond_event, s));
        ++m->cond_gen;
    }
    // the control-frequency token is constant: embed it once (rdt1b.cpp:316)
    SF_TRY(timestep_embed(m, m->fe, c.ctrl_freq, m->f_emb, s));
    // and so are the sampler schedule's timestep tokens (rdt1b.cpp:312-315 at
    // each t of Schedule::linspace, flow_matching.cpp:10-17)
    const std::vector<float> ts = schedule(c.num_steps);
    for (int step = 0; step < c.num_steps; ++step)
        SF_TRY(timestep_embed(m, m->te, timestep_index(c, ts[step]), m->t_emb_steps + (size_t)step * D, s));
    return SF_OK;
}

extern "C" int sf_rdt_set_lang_rows(sf_rdt* m, int32_t rows) {
    if (!m || rows < 1 || rows > m->cfg.lang_max) return SF_EINVAL;
    if (rows == m->lang_rows) return SF_OK;
    m->lang_rows = rows;
    m->infer_cond_valid = false;   // sf_rdt_infer re-encodes with the new rows
    if (m->cfg.batch != 1) return SF_OK;
    // the language GEMMs at M = rows: library-path algorithms chosen now,
    // outside any capture (adaptor 4096 -> D -> D, K/V projection D -> 2D)
    const sf_rdt_config& c = m->cfg;
    const int D = c.hidden;
    const int shapes[3][2] = {{D, c.lang_token_dim}, {D, D}, {2 * D, D}};
    const int widx[3] = {m->la[0], m->la[2], c.layers > 0 ? m->layers[0].ckv_w : m->la[2]};
    for (int j = 0; j < 3; ++j) {
        sf_gemm_desc d{};
        d.M = rows;
        d.N = shapes[j][0];
        d.K = shapes[j][1];
        d.lda = d.K;
        d.a_dtype = SF_BF16;
        d.ldw = d.K;
        d.w_dtype = m->params[widx[j]].dtype;
        SF_TRY(sf_gemm_prepare(&d));
    }
    if (kv_batched(m, 0, rows)) {   // the language blocks' K/V projections as one GEMM
        const sf_gemm_desc d = kv_group_desc(m, 0, nullptr, rows);
        SF_TRY(sf_gemm_prepare(&d));
    }
    return SF_OK;
}

extern "C" int sf_rdt_encode_condition(sf_rdt* m, const void* lang_tokens, const int32_t* lang_len,
                                       const void* img_tokens, const void* state, void* stream) {
    if (!m || !lang_tokens || !lang_len || !img_tokens || !state) return SF_EINVAL;
    const sf_rdt_config& c = m->cfg;
    hipStream_t s = pick_stream(m, stream);
    const int D = c.hidden, B = c.batch;
    // lang_adaptor: mlp2x_gelu 4096 -> D -> D (rdt1b.cpp:118-120, 185), over
    // the L token rows at batch 1
    const int lrows = B == 1 ? m->lang_rows : B * c.lang_max;
    SF_TRY(linear(m, lang_tokens, c.lang_token_dim, lrows, m->la[0], m->la[1], SF_ACT_GELU_TANH, m->ad_h,
                  D, SF_BF16, false, s));
    SF_TRY(linear(m, m->ad_h, D, lrows, m->la[2], m->la[3], SF_ACT_NONE, m->lang_c, D, SF_BF16, false,
                  s));
    // img_adaptor: mlp2x_gelu 1152 -> D -> D (:121-123, 199)
    SF_TRY(linear(m, img_tokens, c.img_token_dim, B * c.img_len, m->ia[0], m->ia[1],
                  SF_ACT_GELU_TANH, m->ad_h, D, SF_BF16, false, s));
    SF_TRY(linear(m, m->ad_h, D, B * c.img_len, m->ia[2], m->ia[3], SF_ACT_NONE, m->img_c, D,
                  SF_BF16, false, s));
    // state token: state_adaptor(cat(state, zeros)) (:202-229)
    // [state | 0] staged on device
    SF_HIP(hipMemsetAsync(m->act_in, 0, (size_t)B * 2 * c.state_dim * 2, s));
    SF_HIP(hipMemcpy2DAsync(m->act_in, (size_t)2 * c.state_dim * 2, state, (size_t)c.state_dim * 2,
                            (size_t)c.state_dim * 2, B, hipMemcpyDeviceToDevice, s));
    SF_TRY(linear(m, m->act_in, 2 * c.state_dim, B, m->sa[0], m->sa[1], SF_ACT_GELU_TANH, m->sa0, D,
                  SF_BF16, false, s));
    SF_TRY(linear(m, m->sa0, D, B, m->sa[2], m->sa[3], SF_ACT_GELU_TANH, m->sa1, D, SF_BF16, false,
                  s));
    SF_TRY(linear(m, m->sa1, D, B, m->sa[4], m->sa[5], SF_ACT_NONE, m->state_tok, D, SF_BF16, false,
                  s));
    // the adaptor outputs are in place: add position embeddings, project K/V
    return sf_rdt_set_condition(m, m->lang_c, lang_len, m->img_c, m->state_tok, stream);
}

extern "C" int sf_rdt_run_blocks(sf_rdt* m, float* x, int32_t first, int32_t count, void* stream) {
    if (!m || !x || first < 0 || count < 0 || first + count > m->cfg.layers) return SF_EINVAL;
    const sf_rdt_config& c = m->cfg;
    hipStream_t s = pick_stream(m, stream);
    SF_TRY(resolve_pv_forms(m));
    const size_t nbytes = (size_t)c.batch * (c.horizon + 3) * c.hidden * 4;
    SF_TRY(refresh_w16(m, s));
    SF_HIP(hipMemcpyAsync(m->x, x, nbytes, hipMemcpyDeviceToDevice, s));
    SF_TRY(entry_norm(m, first, s));
    for (int i = first; i < first + count; ++i) SF_TRY(block_forward(m, i, s));
    SF_HIP(hipMemcpyAsync(x, m->x, nbytes, hipMemcpyDeviceToDevice, s));
    return SF_OK;
}

extern "C" int sf_rdt_denoise_step(sf_rdt* m, const float* x_t, float t, float* velocity,
                                   void* stream) {
    if (!m || !x_t || !velocity) return SF_EINVAL;
    const sf_rdt_config& c = m->cfg;
    hipStream_t s = pick_stream(m, stream);
    SF_TRY(resolve_pv_forms(m));
    SF_TRY(refresh_w16(m, s));
    SF_TRY(step_forward(m, x_t, t, s));
    // last T token rows of each batch element (rdt1b.cpp:362-368)
    SF_HIP(hipMemcpy2DAsync(velocity, (size_t)c.horizon * c.action_dim * 4,
                            m->vel_rows + 3 * c.action_dim, (size_t)(c.horizon + 3) * c.action_dim * 4,
                            (size_t)c.horizon * c.action_dim * 4, c.batch, hipMemcpyDeviceToDevice, s));
    return SF_OK;
}

extern "C" int sf_rdt_sample(sf_rdt* m, float* x, int32_t use_graph, void* stream) {
    if (!m || !x) return SF_EINVAL;
    const sf_rdt_config& c = m->cfg;
    hipStream_t s = pick_stream(m, stream);
    SF_TRY(resolve_pv_forms(m));
    SF_TRY(refresh_w16(m, s));
    const size_t nbytes = (size_t)c.batch * c.horizon * c.action_dim * 4;
    // the initial noise is copied in outside the graph (flow_matching.cpp:49-51)
    SF_HIP(hipMemcpyAsync(m->x_state, x, nbytes, hipMemcpyDeviceToDevice, s));
    if (use_graph) {
        if (m->graph_exec && m->graph_stream != s) release_graph(m);
        if (!m->graph_exec) {
            SF_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
            const int st = sample_body(m, s);
            hipGraph_t g = nullptr;
            const hipError_t e = hipStreamEndCapture(s, &g);
            if (st != SF_OK) {
                if (g) (void)hipGraphDestroy(g);
                return st;
            }
            if (e != hipSuccess || !g) return SF_EDEVICE;
            if (hipGraphInstantiate(&m->graph_exec, g, nullptr, nullptr, 0) != hipSuccess) {
                (void)hipGraphDestroy(g);
                return SF_EDEVICE;
            }
            m->graph = g;
            m->graph_stream = s;
        }
        SF_HIP(hipGraphLaunch(m->graph_exec, s));
    } else {
        SF_TRY(sample_body(m, s));
    }
    SF_HIP(hipMemcpyAsync(x, m->x_state, nbytes, hipMemcpyDeviceToDevice, s));
    return SF_OK;
}

// InferenceEngine::infer (src/engine/inference_engine.cpp:99-175): encode
// the condition when the frame changed (or nothing valid is cached), x_T,
// the Euler loop as one graph replay, the action chunk to the host, and a
// stream synchronisation before returning.  decode_action is the identity
// for RDT-1B (include/servoflow/models/rdt1b/rdt1b.h:35-37).
extern "C" int sf_rdt_infer(sf_rdt* m, uint64_t frame_id, const void* lang_tokens, const int32_t* lang_len,
                            const void* img_tokens, const void* state, uint64_t noise_seed,
                            float* action_out, int32_t* encoded, void* stream) {
    if (!m || !action_out) return SF_EINVAL;
    const sf_rdt_config& c = m->cfg;
    hipStream_t s = pick_stream(m, stream);
    const bool need_encode = !m->infer_cond_valid || m->infer_cond_frame != frame_id;
    if (need_encode) {
        SF_TRY(sf_rdt_encode_condition(m, lang_tokens, lang_len, img_tokens, state, stream));
        m->infer_cond_valid = true;
        m->infer_cond_frame = frame_id;
    }
    if (encoded) *encoded = need_encode ? 1 : 0;
    const int64_t n = (int64_t)c.batch * c.horizon * c.action_dim;
    // x_T ~ N(0, 1), element i from (noise_seed, i); seed 0 keeps the
    // reference's zero placeholder (inference_engine.cpp:133-136)
    if (noise_seed != 0) SF_TRY(sf_init_normal(m->x_infer, SF_F32, n, noise_seed, 1.f, s));
    else SF_TRY(sf_fill_f32(m->x_infer, n, 0.f, s));
    SF_TRY(sf_rdt_sample(m, m->x_infer, 1, s));
    SF_HIP(hipMemcpyAsync(action_out, m->x_infer, (size_t)n * 4, hipMemcpyDeviceToHost, s));
    SF_HIP(hipStreamSynchronize(s));
    return SF_OK;
}

extern "C" int32_t sf_rdt_pv_exact(sf_rdt* m, int32_t layer) {
    if (!m || layer < 0 || layer >= m->cfg.layers) return -1;
    if (resolve_pv_forms(m) != SF_OK) return -1;
    return m->exact_pv[layer];
}
