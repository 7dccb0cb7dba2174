/*
 * sf_hip.h — C-ABI of the MI355X (gfx950) kernel library `libsf_hip_kernels.so`.
 *
 * This is the drop-in boundary for the attention hot path of servoflow's
 * RDT-1B denoising loop.  Every entry point takes plain device pointers,
 * element strides and sizes, runs asynchronously on the given HIP stream,
 * never allocates or synchronises, and returns an `sf_status` code instead of
 * throwing.  All calls are capturable into a hipGraph.
 *
 * Reference interfaces replaced (paths relative to the servoflow tree):
 *   sf_attn_fwd            IBackend::attention
 *                          include/servoflow/backend/backend.h:105-110,
 *                          implemented by CUDABackend::attention
 *                          src/backend/cuda/cuda_backend.cu:470-501 and
 *                          cuda_ops::flash_attention
 *                          src/backend/cuda/ops/attention.cu:183-197.
 *   sf_attn_workspace_bytes the per-call workspace that
 *                          CUDABackend::attention sizes and allocates with
 *                          cudaMallocAsync (cuda_backend.cu:483-490); here the
 *                          caller owns it, so no allocation happens per call.
 *   sf_strerror            the message text of the std::runtime_error /
 *                          std::invalid_argument the reference throws
 *                          (cuda_backend.cu:22-40, 156-161).
 */
#ifndef SF_HIP_H_
#define SF_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  0 is success; errors are negative. */
typedef enum sf_status {
    SF_OK         = 0,
    SF_EINVAL     = -1,  /* bad shape, stride, alignment or argument       */
    SF_ENOTSUP    = -2,  /* valid request this library does not implement  */
    SF_EWORKSPACE = -3,  /* workspace missing or smaller than required     */
    SF_ELAUNCH    = -4,  /* kernel launch failed (hipGetLastError)         */
    SF_EDEVICE    = -5,  /* HIP runtime error outside a launch             */
    SF_ESCRATCH   = -6   /* request exceeds a fixed device scratch buffer  */
} sf_status;

/* Element types.  The numeric values equal servoflow's sf::DType
 * (include/servoflow/core/dtype.h:11-20) so a shim can cast directly. */
typedef enum sf_dtype {
    SF_F32  = 0,
    SF_F16  = 1,
    SF_BF16 = 2,
    SF_I8   = 3,
    SF_I32  = 5
} sf_dtype;

/*
 * Attention descriptor: out = softmax(Q·Kᵀ·scale) · V per (batch, head).
 *
 * Shapes: Q [B,H,Sq,D], K/V [B,H,Sk,D], out [B,H,Sq,D] addressed through
 * element strides (b, h, s); the head dimension d is contiguous (stride 1).
 * Writing out with o_stride = {Sq*H*D, D, H*D} stores [B,Sq,H*D] directly,
 * which is the layout the RDT block's output projection consumes
 * (replaces head_to_seq, src/backend/cuda/ops/split_ops.cuh:168-182).
 *
 * scale == 0 means 1/sqrt(D), as in attention.cu:150.
 * is_causal != 0 keeps key k for query q only when k <= q (top-left
 * alignment, attention.cu:117).
 * kv_valid_len: NULL (every key valid) or a DEVICE pointer to B int32
 * lengths; keys [valid_len[b], Sk) of batch b are ignored.  Lengths are
 * clamped to [0, Sk] on the device; a row with no valid key yields zeros.
 * kv_mask: NULL or a DEVICE pointer to a boolean key-padding mask, one byte
 * per key (nonzero = attend), batch b's row at kv_mask + b * kv_mask_stride
 * bytes (4-byte aligned, stride a multiple of 4, each row readable for Sk
 * rounded up to 4 bytes; bytes past Sk are ignored); combined with
 * kv_valid_len by AND.  This is the [B, Sk] key-padding form the RDT block
 * header documents (include/servoflow/models/rdt1b/dit_block.h:141) and the
 * mask argument of IBackend::attention (backend.h:104) that the reference
 * implementations ignore.
 * num_splits: 0 chooses the split-K factor automatically; n > 0 forces n
 * (at most 64).  Automatic: no split when B*H*ceil(Sq/80) fills the 256
 * CUs, none either when it does not and Sk <= 1024 (the call then runs one
 * workgroup per 16 query rows over all keys), key splits for about one
 * workgroup per CU otherwise.
 * exact_pv: 0 (default) runs the key-split kernel's (Sk > 128) P.V
 * contraction in fp16: a bf16 V converted with rounding to nearest, exact for
 * 2^-14 <= |v| < 2^16 (bf16's 8 significant bits fit fp16's 11; smaller
 * magnitudes round to fp16's subnormal grid, an absolute error of at most
 * 2^-25), and P rounded to the nearest fp16, ~2e-4 mean relative error on
 * the output.  A V element
 * with |v| >= 2^16 converts to +-inf, so the output column (head dim) it
 * belongs to becomes inf or NaN in every row that attends to its key, never
 * a saturated value; the other columns are unaffected.  A NaN or inf in V
 * behaves the same way.  1 keeps V in bf16 and P as a bf16 (hi, lo) pair
 * (~1e-5) for any finite V, at ~15% more time per key tile.
 * scale must be >= 0 (SF_ENOTSUP otherwise).
 *
 * in_dtype: SF_BF16, SF_F16 or SF_F32 for Q, K and V (the reference's
 * dispatch, attention.cu:183-197: fp16 -- its default compute dtype,
 * config.h:57 -- to flash attention, fp32 to the naive kernel).  fp16 runs
 * the same kernels with the fp16 MFMA for S = K.Q^T and V as loaded (exact_pv
 * then carries P as an fp16 hi/lo pair); fp32 runs a kernel on the fp32 MFMA
 * (v_mfma_f32_16x16x4_f32: nothing rounded below fp32; exact_pv ignored).
 * out_dtype: SF_BF16, SF_F16 or SF_F32 (rounded to nearest from fp32).
 *
 * Supported: D == 64, pointers 16-byte aligned, every stride a non-negative
 * multiple of 8 elements, s-strides >= D.
 */
typedef struct sf_attn_desc {
    int32_t B, H, Sq, Sk, D;
    float   scale;
    int32_t in_dtype;
    int32_t out_dtype;
    int32_t is_causal;
    int32_t num_splits;
    const int32_t* kv_valid_len;
    int64_t q_stride[3];
    int64_t k_stride[3];
    int64_t v_stride[3];
    int64_t o_stride[3];
    const uint8_t* kv_mask;
    int64_t kv_mask_stride;
    int32_t exact_pv;
    /* Optional (q_partials != NULL): Q given as the split-K partial sums of
     * its projection instead of q (which may then be NULL), the per-head
     * finish of the reference's q = gemm_bias_act(...), split and
     * apply_qk_norm (dit_block.cu:282-307) done inside the attention:
     * Q[b][h][s][d] = rmsnorm over d of (sum_j q_partials[j][b*Sq + s][n]
     * * q_scale[n] + q_bias[n]) * q_gamma[d], rounded to bf16, n = h*64 + d
     * (q_scale, q_bias, q_gamma each optional; q_eps the norm's epsilon).
     * q_partials: fp32 [q_splits][B*Sq][H*64] (sf_gemm's SF_EPI_PARTIALS
     * output), 1 <= q_splits <= 8, summed in ascending order.  bf16 inputs
     * on the query-block grid only (no key split, B*H*ceil(Sq/80) < 256 and
     * Sk <= 1024; such calls take that grid even for Sk <= 128); other calls
     * return SF_ENOTSUP.
     * Without q_partials, q_gamma and k_gamma (each optional, fp32 [64],
     * 16-byte aligned) apply the reference's per-head RMSNorm
     * (apply_qk_norm, dit_block.cu:185-196 and 262-272, called at 218-220
     * and 306-308; rms_norm_kernel_impl, norm.cuh:89-122) to every Q / K
     * row as it is loaded:
     * row[d] * (1 / sqrt(sum_d row[d]^2 / 64 + q_eps)) * gamma[d], rounded to
     * bf16 -- bit for bit what sf_gemm's per-head epilogue over a bf16
     * product (SF_EPI_HEADS above 160 rows) stores.  With q/k/v and their
     * strides pointing into a projection's 16-bit output (row b*S + s,
     * column section*H*64 + h*64 + d) this takes the place of split_qkv /
     * split_kv + apply_qk_norm.  bf16 or fp16 inputs (the normalised rows
     * are rounded to the input type; SF_ENOTSUP for fp32); k_gamma only on
     * the short-key path (Sk <= 128, no forced split). */
    const float* q_partials;
    int32_t q_splits;
    const float* q_bias;
    const float* q_scale;
    const float* q_gamma;
    float q_eps;
    const float* k_gamma;
    /* q_f16 != 0 (in_dtype SF_BF16, no q_partials): Q is given in fp16
     * while K and V are bf16 -- a projection's fp16 output rows against the
     * bf16 cross-attention K/V cache.  Each Q row is normalised with q_gamma
     * (when set) in fp32 and rounded to bf16 as it is loaded, so the
     * contraction is the bf16 one.  SF_ENOTSUP with another in_dtype or
     * with q_partials. */
    int32_t q_f16;
    /* With q_partials: q_row_ss != NULL says the projection's input rows
     * held x * gamma of a deferred RMSNorm (sf_gemm_desc.norm_ss); Q's row
     * b*Sq + s is then scaled by rsqrt(sum_t q_row_ss[t * B*Sq + b*Sq + s]
     * / q_row_n + q_row_eps) (q_row_tiles <= 64 tiles) after q_scale and
     * before q_bias -- as sf_gemm's a_row_ss does, bit for bit.
     * SF_EINVAL without q_partials. */
    const float* q_row_ss;
    int32_t q_row_tiles;
    int32_t q_row_n;
    float q_row_eps;
    /* v_f16 != 0 (in_dtype SF_BF16, exact_pv 0): V is given in fp16 while Q
     * and K are bf16 -- a cross-attention K/V cache whose V was converted
     * once (sf_bf16_to_f16_below) instead of per tile.  The fast P.V form
     * multiplies fp16 V by P rounded to fp16, exactly as it does after
     * converting a bf16 V itself, so a V converted with the same rounding
     * gives the same bits; the short-key kernel (Sk <= 128) takes fp16 V
     * with P as an fp16 (hi, lo) pair.  SF_ENOTSUP with another in_dtype or
     * with exact_pv. */
    int32_t v_f16;
} sf_attn_desc;

/* Fills a descriptor for contiguous [B,H,S,D] tensors (the layout
 * IBackend::attention documents at backend.h:103). */
void sf_attn_desc_init_bhsd(sf_attn_desc* desc, int32_t B, int32_t H,
                            int32_t Sq, int32_t Sk, int32_t D,
                            int32_t in_dtype, int32_t out_dtype);

/* Bytes of device workspace sf_attn_fwd needs for this descriptor: the
 * split-K partials (fp32 running max, running sum and unnormalised output),
 * 0 when the call needs no split.  Its contents need no initialisation;
 * calls that may run concurrently need separate workspaces. */
size_t sf_attn_workspace_bytes(const sf_attn_desc* desc);

/* Split-K factor sf_attn_fwd will use for this descriptor. */
int32_t sf_attn_num_splits(const sf_attn_desc* desc);

/* Enqueues the attention on `stream` (a hipStream_t; NULL = default). */
int sf_attn_fwd(const sf_attn_desc* desc, const void* q, const void* k,
                const void* v, void* out, void* workspace,
                size_t workspace_bytes, void* stream);

/* Allocation-free form of sf_attn_fwd.  No counterpart in the reference:
 * for callers that cannot allocate device memory (code under hipGraph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * split-K partials go to a fixed device array of
 * SF_ATTN_NOALLOC_SCRATCH_BYTES held by the library on every GPU it runs on
 * until the process ends (looked up on the first call on each device: make
 * that first call outside a capture).  Same results as sf_attn_fwd with a
 * caller workspace.  A call whose partials (sf_attn_workspace_bytes) exceed
 * the array returns SF_ESCRATCH without launching anything; every split
 * count chosen automatically fits, only a large forced num_splits does not.
 * All calls on one GPU share its array and nothing in it needs to start at
 * zero: calls that may overlap on one GPU (different streams, or another
 * thread) race on it and must be serialised by the caller. */
#define SF_ATTN_NOALLOC_SCRATCH_BYTES (8u << 20)
int sf_attn_fwd_noalloc(const sf_attn_desc* desc, const void* q, const void* k,
                        const void* v, void* out, void* stream);

/* ---------------------------------------------------------------------------
 * Projections: C[M,N] = act(A[M,K] . W[N,K]^T + bias[N]).
 *
 * Replaces IBackend::gemm_bias_act as the RDT layers call it (trans_b = true;
 * backend.h:159-183, cuda_backend.cu:337-467; callers dit_block.cu:152-160,
 * 207, 233, 284, 291, 321) and folds in the ops around it:
 *   act: SF_ACT_GELU_TANH is GeluOp, SF_ACT_SILU is SiluOp
 *        (src/backend/cuda/ops/elementwise.cuh:35-68);
 *   epilogue SF_EPI_PLAIN: C (row stride ldc) in c_dtype; accumulate != 0
 *        adds into an fp32 C (the residual adds of dit_block.cu:372-384);
 *   epilogue SF_EPI_HEADS: the N columns are 1..3 sections of H*64 (Q|K|V or
 *        K|V, the order of split_qkv / split_kv, split_ops.cuh:62-84,
 *        210-226); section j goes to head_out[j][b][h][s][d] (bf16, element
 *        strides head_stride[j] = {b, h, s}) with row m = b*S + s (M need
 *        not be a multiple of S: the last batch element may be partial,
 *        e.g. the first L < S rows of one element), after an
 *        RMSNorm over the 64 head dims with head_gamma[j] when that pointer
 *        is non-NULL (q_norm / k_norm, dit_block.cu:219-220, 307-308);
 *   epilogue SF_EPI_ADD_NORM: C (fp32 residual) += result, then
 *        norm_out[m] = C[m] * rsqrt(mean(C[m]^2) + eps) * norm_gamma in
 *        norm_dtype (row stride norm_ldo): the branch add followed by the
 *        next RMSNorm, fused_add_rms_norm (norm.cuh:130-171,
 *        backend.h:127-134) as RDTBlock chains them (dit_block.cu:372-384);
 *        N <= 4096;
 *   w_dtype SF_I8: int8 weights with one fp32 scale per row (w_scale[N]),
 *        the weight-only dequant of quantization.cu:18-51 done in registers.
 * A and W rows must be 16-byte aligned (lda, ldw multiples of 8 elements),
 * K a multiple of 32; bias, w_scale, head_gamma, norm_gamma are fp32;
 * head_out must be 8-byte aligned with strides that are multiples of 4.
 *
 * workspace: scratch of sf_gemm_workspace_bytes().  M <= 160 (N a multiple
 * of 16): fp32 split-K partial sums, which spread one weight matrix over all
 * CUs.  M > 160: the library path -- hipBLASLt writes the fp32 product in
 * chunks of <= 8192 rows into the workspace (plus a bf16 copy of int8
 * weights and hipBLASLt's own scratch) and the epilogue kernels read it.
 * Two library-path cases store a bf16 product instead, with the bias (and
 * the int8 row scale) applied by hipBLASLt, as the reference's cuBLASLt
 * BIAS / GELU_BIAS epilogues return C in bf16 (cuda_backend.cu:414-447):
 *   - SF_EPI_PLAIN into a bf16 C without accumulate, act NONE or GELU_TANH:
 *     hipBLASLt writes C itself (GELU_BIAS for the GELU), one rounding as
 *     in the other paths, no epilogue kernel;
 *   - SF_EPI_HEADS / SF_EPI_ADD_NORM with round_product != 0: the per-head
 *     RMSNorm or the residual add + RMSNorm read bf16(A.W^T + bias) -- the
 *     reference's own storage point (the projection's bf16 output feeds
 *     split_qkv / fused_add_rms_norm) -- instead of the fp32 product.
 * int8 weights above 160 rows with no w_codes16 copy are read directly when
 * the call fits (sf_gemm_int8_direct): K = 2048, N a multiple of 256, ldw a
 * multiple of 16, fp16 activations, act NONE or GELU_TANH, and one of the
 * two 16-bit cases above in fp16 (an fp16 C, or round_product); the codes
 * are widened in registers and the product is stored in fp16 with the row
 * scale, bias and activation applied.
 * Other int8 calls there widen the codes into the workspace on every call.
 * With workspace == NULL a single-pass kernel runs instead and nothing
 * beyond A, W and the outputs is touched.  A non-NULL workspace that is too
 * small is SF_EWORKSPACE.  Calls that may run concurrently need separate
 * workspaces.
 * ------------------------------------------------------------------------- */
typedef enum sf_act { SF_ACT_NONE = 0, SF_ACT_GELU_TANH = 1, SF_ACT_SILU = 2 } sf_act;
typedef enum sf_epilogue {
    SF_EPI_PLAIN = 0,
    SF_EPI_HEADS = 1,
    SF_EPI_ADD_NORM = 2,
    /* The split-K path's fp32 K-slice sums stay in the workspace,
     * [sf_gemm_num_splits][M][N] (no bias, scale, activation; C not
     * written), for a consumer to finish -- the attention's q_partials.
     * Only for calls that run split-K (M <= 160 with a workspace); others
     * return SF_ENOTSUP. */
    SF_EPI_PARTIALS = 3
} sf_epilogue;

typedef struct sf_gemm_desc {
    int32_t M, N, K;
    const void* A;          /* [M][lda] bf16 */
    int64_t lda;
    int32_t a_dtype;
    const void* W;          /* [N][ldw] bf16 or int8 */
    int64_t ldw;
    int32_t w_dtype;
    const float* w_scale;   /* [N] for int8 weights */
    const float* bias;      /* [N] or NULL */
    int32_t act;
    int32_t epilogue;
    void* C;                /* SF_EPI_PLAIN output */
    int64_t ldc;
    int32_t c_dtype;
    int32_t accumulate;
    int32_t H, S;           /* SF_EPI_HEADS: heads per section, rows per batch */
    float eps;
    const float* head_gamma[3];
    void* head_out[3];
    int64_t head_stride[3][3];
    const float* norm_gamma; /* SF_EPI_ADD_NORM */
    void* norm_out;
    int64_t norm_ldo;
    int32_t norm_dtype;
    void* workspace;         /* split-K partial sums, or NULL */
    int64_t workspace_bytes;
    int32_t round_product;   /* M > 160, SF_EPI_HEADS / SF_EPI_ADD_NORM: bf16 product (see above) */
    const void* w_codes16;   /* int8 weights, optional: their codes as bf16 [N][K] (16-byte aligned,
                                sf_int8_codes_to_bf16); the library path reads this copy instead of
                                widening the codes itself on every call.  With w16_f16: an fp16
                                copy [N][K] of the weights (int8 codes or bf16 values,
                                sf_weights_to_f16) */
    int32_t w16_f16;         /* nonzero with a_dtype SF_F16: w_codes16 is the fp16 copy, and the
                                library path (M > 160) multiplies the fp16 activations by it in
                                fp16 -- no rounding of the activations to bf16 -- and its 16-bit
                                products (round_product, and a plain C written by hipBLASLt, which
                                must then be SF_F16) are fp16 (SF_EINVAL when w_codes16 is NULL on
                                this path).  The split-K path (M <= 160) reads the copy instead of
                                W when one is given: the operands it would otherwise form from W in
                                registers, so the same results without the conversion.  The
                                single-pass path reads W itself */
    /* Deferred RMSNorm (split-K path, M <= 160 with a workspace; SF_ENOTSUP
     * elsewhere; N a multiple of 64).  norm_ss (SF_EPI_ADD_NORM): instead of
     * the normalised row, norm_out[m] = C[m] * norm_gamma after the residual
     * add, and norm_ss[t * M + m] = the sum of C[m][n]^2 over the 64 columns
     * n of tile t (N / 64 tiles, fp32, 16-byte aligned) -- the row-wide
     * reduction is left to the consumer, so no workgroup waits for a whole
     * row.  a_row_ss (SF_EPI_PLAIN / SF_EPI_HEADS): A holds such rows; output
     * row m is scaled by rsqrt(sum_t a_row_ss[t * M + m] / a_row_n +
     * a_row_eps) (a_row_tiles tiles, <= 64) after the int8 scale and before
     * the bias: (s a) W^T = s (a W^T), the normalisation of
     * fused_add_rms_norm (norm.cuh:130-171) applied after the product. */
    float* norm_ss;
    const float* a_row_ss;
    int32_t a_row_tiles;
    int32_t a_row_n;
    float a_row_eps;
} sf_gemm_desc;

/* Bytes of workspace sf_gemm needs for this call (0: it always runs
 * single-pass): the split-K partials (M <= 160), or on the library path the
 * product buffer of the epilogue (none when hipBLASLt writes a plain bf16 C
 * itself), the int8 weights' bf16 copy and hipBLASLt's scratch. */
size_t sf_gemm_workspace_bytes(const sf_gemm_desc* desc);

int sf_gemm(const sf_gemm_desc* desc, void* stream);

/* K slices the split-K path uses for this shape (M, N, K, a_dtype), 0 when
 * the call does not run split-K. */
int32_t sf_gemm_num_splits(const sf_gemm_desc* desc);

/* 1 when sf_gemm multiplies this call's int8 weights directly above 160
 * rows (no 16-bit copy: w_codes16 NULL, the shape, types and epilogue
 * listed with the workspace above), else 0; pointers are not inspected.
 * Replaces the dequantize_int8_fp16_kernel pass (quantization.cu:18-51)
 * ahead of gemm_bias_act (cuda_backend.cu:337-467) for those calls. */
int32_t sf_gemm_int8_direct(const sf_gemm_desc* desc);

/* The SF_EPI_HEADS epilogue on a bf16 projection already in memory -- the
 * reference's split_qkv / split_kv followed by apply_qk_norm
 * (split_ops.cuh:62-84, dit_block.cu:185-196, 300-308) in one pass: row m of
 * P [M][ldp] (bias applied) is cut into N / (H*64) <= 3 sections of H heads,
 * each head's 64 values RMS-normalised with head_gamma[j] (when not NULL)
 * and written to head_out[j] at (m / S, h, m % S) with head_stride[j].
 * desc: M, N (a multiple of 64), H, S, eps, head_out, head_gamma,
 * head_stride as for sf_gemm; the GEMM fields are not read.  P 8-byte
 * aligned, ldp >= N a multiple of 4 (16 bytes and 8 take 16-byte loads).
 * Lets a caller run several projections as one GEMM (the runtime's K/V
 * cache: every layer's K/V weights in one matrix) and split per layer. */
int sf_heads_bf16(const sf_gemm_desc* desc, const void* P, int64_t ldp, void* stream);

/* Setup of the library path (M > 160) for this shape, once per shape and
 * process: for the fp32 product and the two bf16 products with bias (plain,
 * GELU) the hipBLASLt algorithm is chosen by timing its first 16
 * candidates on scratch buffers of the shape, each over weight copies
 * totalling 320 MB so that the weights stream from HBM as in a model step
 * (synchronous: allocates, launches on a private stream, frees).  sf_gemm
 * on a shape never prepared takes hipBLASLt's first candidate without
 * timing.  Call this before capturing a graph that contains the call. */
int sf_gemm_prepare(const sf_gemm_desc* desc);

/* Whether sf_gemm_prepare times hipBLASLt's candidates (timed = 1, the
 * default) or takes the first candidate of hipBLASLt's heuristic (0).  The
 * timed pick can differ from one process to the next, and with it the
 * bits of library-path products (M > 160); with 0 every process picks the
 * same algorithm for a given hipBLASLt, GPU and shape, so those products
 * are reproducible bit for bit, at up to ~35% more time per call.  Applies
 * to shapes prepared after the call (a shape keeps the algorithm it was
 * prepared with for the life of the process).  No counterpart in the
 * reference, whose cuBLASLt calls take cuBLASLt's heuristic choice
 * (cuda_backend.cu:414-447).  SF_EINVAL for other values. */
int sf_gemm_set_algo_timing(int32_t timed);

/* Which hipBLASLt algorithm the library path runs for this call's shape and
 * kind (M > 160; the first chunk of <= 8192 rows): *pick = its index in
 * hipBLASLt's heuristic list (0 = the heuristic's first choice),
 * *candidates = the usable candidates, *timed = 1 when the pick came from
 * timing them (sf_gemm_prepare with timing on), 0 otherwise.  SF_ENOTSUP
 * (pick -1) for a shape that is not on the library path or has not been
 * set up yet (sf_gemm_prepare or a first call).  No counterpart in the
 * reference: a record of what ran, for reproducibility reports. */
int sf_gemm_algo_pick(const sf_gemm_desc* desc, int32_t* pick, int32_t* candidates, int32_t* timed);

/* ---------------------------------------------------------------------------
 * Normalisation and dequant.
 * ------------------------------------------------------------------------- */
/* out[r] = x[r] * rsqrt(mean(x[r]^2) + eps) * gamma, fp32 accumulation
 * (rms_norm_kernel_impl, src/backend/cuda/ops/norm.cuh:89-122;
 * IBackend::rms_norm, backend.h:120-122).  x in SF_F32 or SF_BF16, out in
 * SF_BF16 or SF_F32, gamma fp32 [cols]. */
int sf_rmsnorm(const void* x, int32_t x_dtype, int64_t ldx, const float* gamma,
               void* out, int32_t out_dtype, int64_t ldo, int32_t rows,
               int32_t cols, float eps, void* stream);

/* Deferred RMSNorm of fp32 rows x (cols a multiple of 64, rows 16-byte
 * aligned): out[r] = x[r] * gamma (not yet normalised) and ss[t * rows + r]
 * = the sum of x[r][c]^2 over the 64 columns c of tile t, for a consumer
 * that applies rsqrt(sum_t ss / cols + eps) after its contraction
 * (sf_gemm_desc.a_row_ss, sf_attn_desc.q_row_ss) -- rms_norm_kernel_impl
 * (norm.cuh:89-122) with its row-wide step moved into the consumer. */
int sf_rmsnorm_deferred(const float* x, int64_t ldx, const float* gamma, void* out, int32_t out_dtype,
                        int64_t ldo, float* ss, int32_t rows, int32_t cols, void* stream);

/* residual[r] += delta[r]; out[r] = rmsnorm(residual[r]) * gamma
 * (fused_add_rms_norm_kernel, norm.cuh:130-171; IBackend::fused_add_rms_norm,
 * backend.h:127-134).  residual fp32 (kept in fp32 here), delta SF_F32 or
 * SF_BF16, out SF_BF16 or SF_F32. */
int sf_add_rmsnorm(const void* delta, int32_t delta_dtype, float* residual,
                   const float* gamma, void* out, int32_t out_dtype,
                   int32_t rows, int32_t cols, float eps, void* stream);

/* out[i] = float(q[i]) * scale[i / K] (per_channel != 0) or * scale[0],
 * q int8 [N][K] row-major (dequantize_int8_fp16_kernel,
 * src/backend/cuda/ops/quantization.cu:18-51; IBackend::dequantize,
 * backend.h:205-206).  out in SF_F32 or SF_BF16 (the reference writes fp16
 * with an fp16 scale; here the scale is fp32). */
int sf_dequant_int8(const int8_t* q, const float* scale, int32_t per_channel,
                    void* out, int32_t out_dtype, int64_t N, int64_t K,
                    void* stream);

/* Exact bf16 copies of int8 weight codes (no scale: |code| <= 128 fits
 * bf16's 8 significant bits), for up to SF_CODES_MAX_JOBS matrices in one
 * launch: job j widens q [N][ldq] into out [N][K].  The unpack of
 * dequantize_int8_fp16_kernel (quantization.cu:18-51) without its scale
 * multiply; the library path of sf_gemm (M > 160) takes such a copy as
 * w_codes16, so a caller running several int8 projections at a large batch
 * can widen their weights in one pass instead of one pass per call.  ldq
 * and K multiples of 16, pointers 16-byte aligned. */
#define SF_CODES_MAX_JOBS 8
typedef struct sf_codes_job {
    const int8_t* q;
    int64_t ldq;
    void* out;
    int32_t N, K;
} sf_codes_job;
int sf_int8_codes_to_bf16(const sf_codes_job* jobs, int32_t count, void* stream);

/* fp16 copies of projection weights for the library path's fp16 products
 * (sf_gemm_desc.w16_f16): job j converts w [N][ldw] -- int8 codes (exact,
 * no scale: the row scale stays with the GEMM) or bf16 values (rounded to
 * the nearest fp16: exact for 2^-14 <= |w| < 65520, within 2^-25 below,
 * +-inf at or above 65520) -- into out [N][K], up to SF_CODES_MAX_JOBS
 * matrices per launch.  K a multiple of 16, rows 16-byte aligned. */
typedef struct sf_w16_job {
    const void* w;
    int32_t w_dtype;   /* SF_I8 or SF_BF16 */
    int64_t ldw;       /* elements */
    void* out;
    int32_t N, K;
} sf_w16_job;
int sf_weights_to_f16(const sf_w16_job* jobs, int32_t count, void* stream);

/* Static text for a status code. */
const char* sf_strerror(int status);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* SF_HIP_H_ */
