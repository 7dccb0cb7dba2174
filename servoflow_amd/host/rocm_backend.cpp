// RocmBackend::attention over sf_attn_fwd (see rocm_backend.h).
//
// Mirrors CUDABackend::attention (src/backend/cuda/cuda_backend.cu:470-501):
// device checks, a workspace, one kernel launch on the caller's stream; with
// the differences that each stream's workspace persists across calls instead
// of a per-call cudaMallocAsync / cudaFreeAsync (:483-490), and that the mask
// is applied instead of ignored.
#include "rocm_backend.h"

#include <hip/hip_runtime.h>

#include <stdexcept>
#include <string>

#include "sf_hip.h"

namespace sf_amd {

size_t dtype_size(DType dt) {
    switch (dt) {
        case DType::Float32: return 4;
        case DType::Float16: return 2;
        case DType::BFloat16: return 2;
        case DType::Int8: return 1;
        case DType::Int4: return 1;
        case DType::Int32: return 4;
        case DType::Bool: return 1;
    }
    return 0;
}

int64_t TensorRef::numel() const {
    int64_t n = 1;
    for (int64_t s : shape) n *= s;
    return n;
}

TensorRef TensorRef::contiguous(void* data, DType dtype, std::vector<int64_t> shape, bool on_device) {
    TensorRef t;
    t.data = data;
    t.dtype = dtype;
    t.shape = std::move(shape);
    t.strides.assign(t.shape.size(), 0);
    int64_t s = (int64_t)dtype_size(dtype);
    for (int i = (int)t.shape.size() - 1; i >= 0; --i) {
        t.strides[i] = s;
        s *= t.shape[i];
    }
    t.on_device = on_device;
    return t;
}

namespace {

[[noreturn]] void bad(const std::string& what) {
    throw std::invalid_argument("RocmBackend::attention: " + what);
}

int32_t sf_type(DType dt) {
    switch (dt) {
        case DType::Float32: return SF_F32;
        case DType::Float16: return SF_F16;
        case DType::BFloat16: return SF_BF16;
        default: return -1;
    }
}

// Element strides (b, h, s) of a 4-D BHSD tensor with a contiguous last dim.
void elem_strides(const TensorRef& t, const char* name, int64_t out[3]) {
    if (t.ndim() != 4) bad(std::string(name) + " must be 4-D [B,H,S,D]");
    const int64_t es = (int64_t)dtype_size(t.dtype);
    if (t.strides.size() != 4 || t.strides[3] != es)
        bad(std::string(name) + " must be contiguous along the head dim");
    for (int i = 0; i < 3; ++i) {
        if (t.strides[i] % es) bad(std::string(name) + " strides must be whole elements");
        out[i] = t.strides[i] / es;
    }
}

void check_status(int st) {
    if (st == SF_OK) return;
    const std::string msg = std::string("RocmBackend::attention: ") + sf_strerror(st);
    if (st == SF_EINVAL || st == SF_ENOTSUP) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

// Fills the mask fields of the descriptor from the reference's mask forms.
void apply_mask(const TensorRef& m, int64_t B, int64_t Sk, sf_attn_desc& d) {
    if (!m.on_device) bad("mask must be on the device");
    if (m.dtype == DType::Int32) {
        if (m.numel() != B) bad("an Int32 mask holds one valid key length per batch element");
        if (m.strides.empty() || m.strides.back() != 4) bad("Int32 valid lengths must be contiguous");
        d.kv_valid_len = static_cast<const int32_t*>(m.data);
        return;
    }
    if (m.dtype == DType::Bool || m.dtype == DType::Int8) {
        // [B, Sk] or [B, 1, 1, Sk]: one key-padding row per batch element
        const bool two_d = m.ndim() == 2 && m.shape[0] == B && m.shape[1] == Sk;
        const bool four_d = m.ndim() == 4 && m.shape[0] == B && m.shape[1] == 1 && m.shape[2] == 1 &&
                            m.shape[3] == Sk;
        if (!two_d && !four_d)
            bad("unsupported mask: a Bool mask must be a key-padding mask [B,Sk] or [B,1,1,Sk]");
        if (m.strides.back() != 1) bad("a key-padding mask must be contiguous along Sk");
        d.kv_mask = static_cast<const uint8_t*>(m.data);
        d.kv_mask_stride = m.strides[0];
        return;
    }
    bad("unsupported mask: additive float masks are not implemented (use a Bool key-padding mask)");
}

}  // namespace

RocmBackend::~RocmBackend() {
    for (auto& kv : ws_)
        if (kv.second.ptr) (void)hipFree(kv.second.ptr);
}

size_t RocmBackend::attention_workspace_bytes(const TensorRef& Q, const TensorRef& K) {
    if (Q.ndim() != 4 || K.ndim() != 4) return 0;
    sf_attn_desc d;
    // the partials' size does not depend on the element type
    sf_attn_desc_init_bhsd(&d, (int32_t)Q.shape[0], (int32_t)Q.shape[1], (int32_t)Q.shape[2],
                           (int32_t)K.shape[2], (int32_t)Q.shape[3], SF_BF16, SF_BF16);
    return sf_attn_workspace_bytes(&d);
}

void RocmBackend::grow(Workspace& ws, size_t bytes, StreamHandle stream) {
    if (bytes <= ws.bytes) return;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess)
        throw std::runtime_error("RocmBackend::attention: hipStreamIsCapturing failed");
    if (cs != hipStreamCaptureStatusNone)
        throw std::runtime_error(
            "RocmBackend::attention: workspace too small inside graph capture; call "
            "reserve_attention_workspace() for this stream before capturing");
    if (ws.ptr) {
        // earlier calls queued on this stream may still read the old buffer
        if (hipStreamSynchronize(s) != hipSuccess)
            throw std::runtime_error("RocmBackend: hipStreamSynchronize failed");
        if (hipFree(ws.ptr) != hipSuccess) throw std::runtime_error("RocmBackend: hipFree failed");
        ws.ptr = nullptr;
        ws.bytes = 0;
    }
    if (hipMalloc(&ws.ptr, bytes) != hipSuccess) {
        ws.ptr = nullptr;
        throw std::runtime_error("RocmBackend: workspace allocation failed");
    }
    ws.bytes = bytes;
}

void RocmBackend::reserve_attention_workspace(size_t bytes, StreamHandle stream) {
    std::lock_guard<std::mutex> lock(mu_);
    grow(ws_[stream], bytes, stream);
}

void RocmBackend::attention(const TensorRef& Q, const TensorRef& K, const TensorRef& V,
                            TensorRef& out, const TensorRef* mask, float scale, bool is_causal,
                            StreamHandle stream) {
    if (!Q.on_device || !K.on_device || !V.on_device || !out.on_device)
        bad("all tensors must reside on the ROCm device");
    if (Q.ndim() != 4 || K.ndim() != 4 || V.ndim() != 4 || out.ndim() != 4)
        bad("expected Q [B,H,S,D], K/V [B,H,Sk,D], out [B,H,S,D]");
    const int64_t B = Q.shape[0], H = Q.shape[1], S = Q.shape[2], D = Q.shape[3], Sk = K.shape[2];
    if (K.shape != std::vector<int64_t>{B, H, Sk, D} || V.shape != K.shape || out.shape != Q.shape)
        bad("shape mismatch between Q, K, V and out");
    if (Q.dtype != K.dtype || Q.dtype != V.dtype) bad("Q, K and V must share a dtype");
    if (sf_type(Q.dtype) < 0) bad("Q, K and V must be Float32, Float16 or BFloat16");
    if (sf_type(out.dtype) < 0) bad("out must be Float32, Float16 or BFloat16");

    sf_attn_desc d;
    sf_attn_desc_init_bhsd(&d, (int32_t)B, (int32_t)H, (int32_t)S, (int32_t)Sk, (int32_t)D,
                           sf_type(Q.dtype), sf_type(out.dtype));
    elem_strides(Q, "Q", d.q_stride);
    elem_strides(K, "K", d.k_stride);
    elem_strides(V, "V", d.v_stride);
    elem_strides(out, "out", d.o_stride);
    d.scale = scale;
    d.is_causal = is_causal ? 1 : 0;
    d.exact_pv = precision_ == AttentionPrecision::Exact ? 1 : 0;
    if (mask) apply_mask(*mask, B, Sk, d);

    std::lock_guard<std::mutex> lock(mu_);
    Workspace& ws = ws_[stream];
    grow(ws, sf_attn_workspace_bytes(&d), stream);
    check_status(sf_attn_fwd(&d, Q.data, K.data, V.data, out.data, ws.ptr, ws.bytes, stream));
}

}  // namespace sf_amd
