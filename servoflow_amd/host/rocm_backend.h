// RocmBackend: the reference's IBackend::attention operator
// (include/servoflow/backend/backend.h:105-110) as a C++ class over the
// C-ABI of libsf_hip_kernels.so (sf_attn_fwd, include/sf_hip.h).
//
// This is the layer a servoflow maintainer binds to: it takes tensors the way
// sf::Tensor describes them (shape, dtype, BYTE strides as in
// include/servoflow/core/tensor.h:43,121-127, raw data pointer, device), keeps
// the operator's argument meaning (scale 0 -> 1/sqrt(D), optional mask,
// is_causal, opaque stream handle) and reports failures with the reference's
// exception types: std::invalid_argument for bad arguments or unsupported
// configurations (cuda_backend.cu:156-161), std::runtime_error for runtime
// failures (cuda_backend.cu:22-40).
//
// Mask forms (the reference documents an additive [B,1,S,Sk] mask at
// backend.h:104 and a key-padding mask at
// include/servoflow/models/rdt1b/dit_block.h:141, and ignores both):
//   nullptr                          all keys attend
//   Int32 with B elements            per-batch valid key lengths
//   Bool / Int8 [B, Sk] or [B,1,1,Sk] key-padding mask (nonzero = attend),
//                                    contiguous along Sk, rows readable for
//                                    Sk rounded up to 4 bytes
//   Float32 / Float16 / BFloat16     the additive mask of backend.h:104,
//     [B,1,1,Sk] or [B,1,S,Sk]       softmax(Q K^T * scale + mask): read on
//                                    the host (synchronously; not inside a
//                                    graph capture) and applied as its
//                                    key-padding form -- per batch element
//                                    every row the same, each entry either
//                                    the row's maximum (kept) or at least
//                                    5000 below it (-1e4, -inf: dropped,
//                                    its weight underflows to 0); a row of
//                                    one value keeps every key
//   anything else                    std::invalid_argument
//
// Thread-compatible like the reference (backend.h:35-42): a stream must not
// be shared across threads.  Each stream gets its own split-K workspace (so
// calls on different streams never share partials), guarded by a mutex; a
// stream's workspace grows on demand outside graph capture (after that
// stream's queued work has finished); before capturing, size it with
// reserve_attention_workspace() for the capturing stream.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <mutex>
#include <vector>

namespace sf_amd {

// Values of sf::DType (include/servoflow/core/dtype.h:11-20).
enum class DType : uint8_t {
    Float32 = 0,
    Float16 = 1,
    BFloat16 = 2,
    Int8 = 3,
    Int4 = 4,
    Int32 = 5,
    Bool = 6,
};

using StreamHandle = void*;   // hipStream_t (backend.h:17)

// Non-owning view of a tensor: what sf::Tensor exposes through shape(),
// dtype(), strides() (bytes), raw_data_ptr() and is_cuda().
struct TensorRef {
    void* data = nullptr;
    DType dtype = DType::Float32;
    std::vector<int64_t> shape;
    std::vector<int64_t> strides;   // bytes per step of each dim
    bool on_device = false;

    int64_t ndim() const { return (int64_t)shape.size(); }
    int64_t numel() const;
    // Contiguous row-major view of device memory.
    static TensorRef contiguous(void* data, DType dtype, std::vector<int64_t> shape,
                                bool on_device = true);
};

size_t dtype_size(DType dt);

// Precision of the P.V contraction for 16-bit inputs.  Exact (the default):
// V in its input type and P carried as a (hi, lo) pair, finite for any
// finite V, like the reference's fp32 naive kernel.  Fast: P rounded to fp16
// (~2e-4 relative error); a BFloat16 V is then converted to fp16, so a V
// element with |v| >= 2^16 makes its output column inf/NaN (the range of the
// reference's fp16 flash-attention path, attention.cu:29-80).  Float32
// inputs ignore this (fp32 products throughout).
enum class AttentionPrecision { Exact, Fast };

class RocmBackend {
public:
    explicit RocmBackend(AttentionPrecision precision = AttentionPrecision::Exact)
        : precision_(precision) {}
    ~RocmBackend();
    RocmBackend(const RocmBackend&) = delete;
    RocmBackend& operator=(const RocmBackend&) = delete;

    // out = softmax(Q K^T * scale [masked]) V per (b, h).
    // Q [B,H,S,D], K/V [B,H,Sk,D] all Float32, Float16 or BFloat16 (one
    // dtype: Float32 is the reference's fp32 path, attention.cu:183-197);
    // out [B,H,S,D] Float32, Float16 or BFloat16 (any strides with a
    // contiguous head dim, e.g. a [B,S,H,D] buffer viewed as BHSD).  D = 64.
    void attention(const TensorRef& Q, const TensorRef& K, const TensorRef& V, TensorRef& out,
                   const TensorRef* mask = nullptr, float scale = 0.f, bool is_causal = false,
                   StreamHandle stream = nullptr);

    // Makes sure `stream`'s split-K workspace holds at least `bytes`
    // (allocates now, outside any capture).  attention_workspace_bytes()
    // gives the size a call needs.
    void reserve_attention_workspace(size_t bytes, StreamHandle stream = nullptr);
    static size_t attention_workspace_bytes(const TensorRef& Q, const TensorRef& K);

    AttentionPrecision precision() const { return precision_; }

private:
    struct Workspace {
        void* ptr = nullptr;
        size_t bytes = 0;
        void* mask = nullptr;   // key-padding form of an additive mask
        size_t mask_bytes = 0;
    };
    // Grows ws to `bytes` outside capture; mu_ held.
    void grow(Workspace& ws, size_t bytes, StreamHandle stream);
    // The key-padding form ([B][Sk rounded up to 4] bytes) of an additive
    // mask; std::invalid_argument for one that has none.
    static std::vector<uint8_t> additive_to_keep(const TensorRef& m, int64_t B, int64_t Sq, int64_t Sk,
                                                 StreamHandle stream);

    AttentionPrecision precision_;
    std::mutex mu_;
    std::map<StreamHandle, Workspace> ws_;
};

}  // namespace sf_amd
