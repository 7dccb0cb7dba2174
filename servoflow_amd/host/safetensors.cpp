// SafeTensors checkpoints for the RDT-1B runtime (libsf_rdt.so).
//
// Native restatement of the reference's loader path:
//   SafeTensorsLoader::parse_header / inspect / load
//     (src/loader/safetensors.cpp:62-160): 8-byte little-endian header
//     length, JSON header {name: {dtype, shape, data_offsets}}, optional
//     "__metadata__", data section after the header;
//   load_weight_from_map (:166-190): host tensor -> device tensor of the
//     model's dtype;
//   remap_key (tools/convert/hf_to_servoflow.py:41-65): HuggingFace names
//     lose a leading "model.", EMA and optimizer entries are skipped.
// The file is memory-mapped (as the reference does) and each tensor is
// converted on the host into the parameter's storage type (fp32, bf16 by
// round-to-nearest-even, or int8 rows quantised as sf_init_int8_rows does),
// then copied to the device.  The header parser (a small recursive descent
// over the JSON subset the format uses) is in st_format.cpp.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "sf_hip.h"
#include "sf_rdt.h"
#include "rdt_internal.h"
#include "st_format.h"

using namespace sf_amd::st;

extern "C" int sf_rdt_load_safetensors(sf_rdt* m, const char* path, int32_t flags, int32_t* loaded) {
    if (!m || !path) return SF_EINVAL;
    if (loaded) *loaded = 0;
    sf_rdt_set_error(m, "");
    Mapped f(path);
    if (!f.data) {
        sf_rdt_set_error(m, std::string("cannot open or map ") + path);
        return SF_EINVAL;
    }
    std::vector<Tensor> ts;
    uint64_t off = 0;
    std::string err;
    if (!parse_header(f.data, f.size, ts, &off, err)) {
        sf_rdt_set_error(m, "safetensors header: " + err);
        return SF_EINVAL;
    }
    const int32_t np = sf_rdt_num_params(m);
    std::vector<char> seen(np, 0);
    std::vector<float> vals;
    int32_t n = 0;
    sf_rdt_weights_changed(m);   // parameters are overwritten from here on
    for (const Tensor& t : ts) {
        const std::string key = remap_key(t.name);
        if (key.empty()) continue;
        const int32_t idx = sf_rdt_find_param(m, key.c_str());
        if (idx < 0) continue;   // not part of this model (action_norm stats, encoders, ...)
        const char* pname = nullptr;
        int32_t pdt = 0, pnd = 0;
        int64_t pshape[4];
        (void)sf_rdt_param_info(m, idx, &pname, &pdt, &pnd, pshape);
        std::vector<int64_t> ps(pshape, pshape + pnd);
        if (!same_shape(ps, t.shape)) {
            sf_rdt_set_error(m, "shape mismatch for " + key);
            return SF_EINVAL;
        }
        if (t.dtype != SF_F32 && t.dtype != SF_F16 && t.dtype != SF_BF16) {
            sf_rdt_set_error(m, "unsupported dtype for " + key + " (F32, F16 and BF16 are read)");
            return SF_ENOTSUP;
        }
        size_t numel = 1;
        for (int64_t d : t.shape) numel *= (size_t)d;
        if (t.end - t.begin != numel * dtype_bytes(t.dtype) || off + t.end > f.size) {
            sf_rdt_set_error(m, "data range of " + key + " does not match its shape or the file");
            return SF_EINVAL;
        }
        to_f32(f.data + off + t.begin, t.dtype, numel, vals);
        void* dst = sf_rdt_param_data(m, idx);
        hipError_t he = hipSuccess;
        if (pdt == SF_F32) {
            he = hipMemcpy(dst, vals.data(), numel * 4, hipMemcpyHostToDevice);
        } else if (pdt == SF_BF16) {
            std::vector<uint16_t> b(numel);
            for (size_t i = 0; i < numel; ++i) b[i] = f32_to_bf16(vals[i]);
            he = hipMemcpy(dst, b.data(), numel * 2, hipMemcpyHostToDevice);
        } else {   // int8 rows: scale = max|w| / 127, q = clamp(rint(w / scale))
            const int64_t rows = pshape[0], cols = (int64_t)(numel / (size_t)rows);
            std::vector<int8_t> q(numel);
            std::vector<float> sc(rows);
            for (int64_t r = 0; r < rows; ++r) {
                float amax = 0.f;
                for (int64_t c = 0; c < cols; ++c) amax = std::fmax(amax, std::fabs(vals[r * cols + c]));
                const float s = amax > 0.f ? amax / 127.f : 1.f;
                sc[r] = s;
                for (int64_t c = 0; c < cols; ++c) {
                    float v = std::rint(vals[r * cols + c] / s);
                    v = std::fmin(127.f, std::fmax(-127.f, v));
                    q[r * cols + c] = (int8_t)v;
                }
            }
            he = hipMemcpy(dst, q.data(), numel, hipMemcpyHostToDevice);
            if (he == hipSuccess)
                he = hipMemcpy(sf_rdt_param_scale(m, idx), sc.data(), rows * 4, hipMemcpyHostToDevice);
        }
        if (he != hipSuccess) {
            sf_rdt_set_error(m, "device copy failed for " + key);
            return SF_EDEVICE;
        }
        if (!seen[idx]) ++n;
        seen[idx] = 1;
    }
    if (loaded) *loaded = n;
    if (!(flags & SF_LOAD_PARTIAL)) {
        for (int32_t i = 0; i < np; ++i) {
            if (!seen[i]) {
                const char* pname = nullptr;
                (void)sf_rdt_param_info(m, i, &pname, nullptr, nullptr, nullptr);
                sf_rdt_set_error(m, std::string("missing key '") + pname + "'");
                return SF_EINVAL;   // load_weight_from_map throws on a missing key (:171-172)
            }
        }
    }
    return SF_OK;
}
