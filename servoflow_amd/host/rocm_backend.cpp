// RocmBackend::attention over sf_attn_fwd (see rocm_backend.h).
//
// Mirrors CUDABackend::attention (src/backend/cuda/cuda_backend.cu:470-501):
// device checks, a workspace, one kernel launch on the caller's stream; with
// the differences that each stream's workspace persists across calls instead
// of a per-call cudaMallocAsync / cudaFreeAsync (:483-490), and that the mask
// is applied instead of ignored.
#include "rocm_backend.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
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

float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const int e = (h >> 10) & 31;
    uint32_t m = h & 0x3ffu;
    uint32_t bits;
    if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {   // subnormal: normalise
            int ee = -1;
            do {
                ++ee;
                m <<= 1;
            } while (!(m & 0x400u));
            bits = sign | ((uint32_t)(127 - 15 - ee) << 23) | ((m & 0x3ffu) << 13);
        }
    } else {
        bits = sign | ((uint32_t)(e - 15 + 127) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

}  // namespace

// An additive mask [B,1,1,Sk] or [B,1,Sq,Sk] as the key-padding form the
// kernels apply.  softmax(s + m) over a row equals softmax(s) over the keys
// whose m equals the row's maximum M whenever every other key has
// m <= M - 5000: those keys' weights exp(s_k + m_k - max) underflow to
// exactly 0 in fp32 (while the raw scores of the row span less than ~4800;
// -1e4 -- -9984 in bf16 --, -1e9 and -inf all qualify), and the common
// offset M of the kept keys cancels.  So per batch element every row must
// be the same and hold only M and values <= M - 5000; a row that is all
// one value keeps every key, as the additive form does.  Anything else (a
// bias between -5000 and the maximum, NaN,
// rows that differ per query) has no key-padding equivalent:
// std::invalid_argument.  The mask is read on the host: not allowed while
// the stream is being captured.
std::vector<uint8_t> RocmBackend::additive_to_keep(const TensorRef& m, int64_t B, int64_t Sq, int64_t Sk,
                                                   StreamHandle stream) {
    const bool key_only = m.ndim() == 4 && m.shape[0] == B && m.shape[1] == 1 && m.shape[2] == 1 && m.shape[3] == Sk;
    const bool per_query = m.ndim() == 4 && m.shape[0] == B && m.shape[1] == 1 && m.shape[2] == Sq && m.shape[3] == Sk;
    if (!key_only && !per_query) bad("an additive mask must be [B,1,1,Sk] or [B,1,S,Sk]");
    const int64_t es = (int64_t)dtype_size(m.dtype);
    if (m.strides.size() != 4 || m.strides[3] != es) bad("an additive mask must be contiguous along Sk");
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess)
        throw std::runtime_error("RocmBackend::attention: hipStreamIsCapturing failed");
    if (cs != hipStreamCaptureStatusNone)
        bad("an additive float mask is read on the host and cannot be used inside graph capture; "
            "pass its Bool key-padding form instead");
    const int64_t rows = key_only ? 1 : Sq;
    std::vector<char> host((size_t)(Sk * es));
    std::vector<float> row((size_t)Sk);
    std::vector<uint8_t> keep((size_t)(B * ((Sk + 3) & ~int64_t(3))), 0);
    const int64_t ld = (Sk + 3) & ~int64_t(3);
    for (int64_t b = 0; b < B; ++b) {
        std::vector<float> first;
        for (int64_t r = 0; r < rows; ++r) {
            const char* src = static_cast<const char*>(m.data) + b * m.strides[0] + r * m.strides[2];
            if (hipMemcpyAsync(host.data(), src, host.size(), hipMemcpyDeviceToHost, s) != hipSuccess ||
                hipStreamSynchronize(s) != hipSuccess)
                throw std::runtime_error("RocmBackend::attention: reading the mask failed");
            for (int64_t k = 0; k < Sk; ++k) {
                float v;
                if (m.dtype == DType::Float32) {
                    std::memcpy(&v, host.data() + 4 * k, 4);
                } else {
                    uint16_t h;
                    std::memcpy(&h, host.data() + 2 * k, 2);
                    if (m.dtype == DType::BFloat16) {
                        const uint32_t bits = (uint32_t)h << 16;
                        std::memcpy(&v, &bits, 4);
                    } else {
                        v = half_to_float(h);
                    }
                }
                if (std::isnan(v) || v == INFINITY) bad("an additive mask holds NaN or +inf");
                row[(size_t)k] = v;
            }
            if (r == 0) {
                first = row;
            } else if (row != first) {
                bad("an additive mask that differs between query rows has no key-padding form");
            }
        }
        float mx = -INFINITY;
        for (float v : first) mx = std::max(mx, v);
        for (int64_t k = 0; k < Sk; ++k) {
            const float v = first[(size_t)k];
            if (v == mx) {
                keep[(size_t)(b * ld + k)] = 1;
            } else if (!(v <= mx - 5000.f)) {
                bad("an additive mask entry is neither the row's maximum nor 5000 or more below it");
            }
        }
    }
    return keep;
}

namespace {

// Fills the mask fields of the descriptor from the reference's mask forms
// (an additive float mask arrives here already as its key-padding form).
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
    bad("unsupported mask dtype (Int32 lengths, Bool / Int8 key padding, or an additive float mask)");
}

}  // namespace

RocmBackend::~RocmBackend() {
    for (auto& kv : ws_) {
        if (kv.second.ptr) (void)hipFree(kv.second.ptr);
        if (kv.second.mask) (void)hipFree(kv.second.mask);
    }
}

size_t RocmBackend::attention_workspace_bytes(const TensorRef& Q, const TensorRef& K) {
    if (Q.ndim() != 4 || K.ndim() != 4 || sf_type(Q.dtype) < 0) return 0;
    sf_attn_desc d;
    // the split count (and with it the partials' size) depends on the
    // element type: Float32 takes key splits where 16-bit types run one
    // workgroup per query block
    sf_attn_desc_init_bhsd(&d, (int32_t)Q.shape[0], (int32_t)Q.shape[1], (int32_t)Q.shape[2],
                           (int32_t)K.shape[2], (int32_t)Q.shape[3], sf_type(Q.dtype), sf_type(Q.dtype));
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
    const bool additive = mask && (mask->dtype == DType::Float32 || mask->dtype == DType::Float16 ||
                                   mask->dtype == DType::BFloat16);
    std::vector<uint8_t> keep;
    if (additive) {
        if (!mask->on_device) bad("mask must be on the device");
        keep = additive_to_keep(*mask, B, S, Sk, stream);
    } else if (mask) {
        apply_mask(*mask, B, Sk, d);
    }

    std::lock_guard<std::mutex> lock(mu_);
    Workspace& ws = ws_[stream];
    if (additive) {   // the key-padding form goes to this stream's mask buffer
        if (keep.size() > ws.mask_bytes) {
            if (hipStreamSynchronize(static_cast<hipStream_t>(stream)) != hipSuccess)
                throw std::runtime_error("RocmBackend: hipStreamSynchronize failed");
            if (ws.mask) (void)hipFree(ws.mask);
            ws.mask = nullptr;
            ws.mask_bytes = 0;
            if (hipMalloc(&ws.mask, keep.size()) != hipSuccess) {
                ws.mask = nullptr;
                throw std::runtime_error("RocmBackend: mask buffer allocation failed");
            }
            ws.mask_bytes = keep.size();
        }
        // synchronous: the host vector is gone when this call returns, and
        // an earlier call on the stream may still read the buffer
        if (hipMemcpyAsync(ws.mask, keep.data(), keep.size(), hipMemcpyHostToDevice,
                           static_cast<hipStream_t>(stream)) != hipSuccess ||
            hipStreamSynchronize(static_cast<hipStream_t>(stream)) != hipSuccess)
            throw std::runtime_error("RocmBackend: uploading the key-padding mask failed");
        d.kv_mask = static_cast<const uint8_t*>(ws.mask);
        d.kv_mask_stride = (Sk + 3) & ~int64_t(3);
    }
    grow(ws, sf_attn_workspace_bytes(&d), stream);
    check_status(sf_attn_fwd(&d, Q.data, K.data, V.data, out.data, ws.ptr, ws.bytes, stream));
}

}  // namespace sf_amd
