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
    SF_EDEVICE    = -5   /* HIP runtime error outside a launch             */
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
 * num_splits: 0 chooses the split-K factor automatically; n > 0 forces n
 * (at most 64).
 * scale must be >= 0 (SF_ENOTSUP otherwise).
 *
 * Supported: in_dtype SF_BF16, out_dtype SF_BF16 or SF_F32, D == 64,
 * pointers 16-byte aligned, s/h/b strides multiples of 8 elements.
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

/* Static text for a status code. */
const char* sf_strerror(int status);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* SF_HIP_H_ */
