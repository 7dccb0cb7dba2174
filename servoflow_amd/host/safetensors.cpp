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
// then copied to the device.  The JSON header parser is a small recursive
// descent over the subset the format uses.
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "sf_hip.h"
#include "sf_rdt.h"
#include "rdt_internal.h"

namespace {

struct StTensor {
    std::string name;
    int32_t dtype = -1;   // SF_F32 / SF_F16 / SF_BF16 / SF_I8 / SF_I32, -1 unknown
    std::vector<int64_t> shape;
    uint64_t begin = 0, end = 0;
};

// ---- JSON subset -----------------------------------------------------------
struct Json {
    const char* p;
    const char* e;
    bool ok = true;

    void ws() {
        while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
    }
    bool eat(char c) {
        ws();
        if (p < e && *p == c) {
            ++p;
            return true;
        }
        return false;
    }
    void fail() { ok = false; p = e; }

    static void put_utf8(std::string& s, uint32_t cp) {
        if (cp < 0x80) {
            s += (char)cp;
        } else if (cp < 0x800) {
            s += (char)(0xC0 | (cp >> 6));
            s += (char)(0x80 | (cp & 0x3F));
        } else {
            s += (char)(0xE0 | (cp >> 12));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        }
    }
    std::string str() {
        std::string s;
        if (!eat('"')) { fail(); return s; }
        while (p < e && *p != '"') {
            if (*p == '\\') {
                if (++p >= e) { fail(); return s; }
                const char c = *p++;
                switch (c) {
                    case '"': s += '"'; break;
                    case '\\': s += '\\'; break;
                    case '/': s += '/'; break;
                    case 'b': s += '\b'; break;
                    case 'f': s += '\f'; break;
                    case 'n': s += '\n'; break;
                    case 'r': s += '\r'; break;
                    case 't': s += '\t'; break;
                    case 'u': {
                        if (e - p < 4) { fail(); return s; }
                        uint32_t cp = 0;
                        for (int i = 0; i < 4; ++i) {
                            const char h = *p++;
                            cp <<= 4;
                            if (h >= '0' && h <= '9') cp |= (uint32_t)(h - '0');
                            else if (h >= 'a' && h <= 'f') cp |= (uint32_t)(h - 'a' + 10);
                            else if (h >= 'A' && h <= 'F') cp |= (uint32_t)(h - 'A' + 10);
                            else { fail(); return s; }
                        }
                        put_utf8(s, cp);
                        break;
                    }
                    default: fail(); return s;
                }
            } else {
                s += *p++;
            }
        }
        if (p >= e) { fail(); return s; }
        ++p;   // closing quote
        return s;
    }
    bool integer(int64_t* out) {
        ws();
        const char* q = p;
        bool neg = false;
        if (q < e && *q == '-') { neg = true; ++q; }
        if (q >= e || *q < '0' || *q > '9') return false;
        uint64_t v = 0;
        while (q < e && *q >= '0' && *q <= '9') {
            v = v * 10 + (uint64_t)(*q - '0');
            if (v > (1ull << 62)) return false;
            ++q;
        }
        if (q < e && (*q == '.' || *q == 'e' || *q == 'E')) return false;
        p = q;
        *out = neg ? -(int64_t)v : (int64_t)v;
        return true;
    }
    // Skips any JSON value (metadata is ignored).  Nesting deeper than
    // kMaxDepth is a header error, so a hostile header cannot exhaust the
    // stack through the recursion.
    static constexpr int kMaxDepth = 64;
    void skip(int depth = 0) {
        ws();
        if (p >= e || depth >= kMaxDepth) { fail(); return; }
        if (*p == '"') { (void)str(); return; }
        if (*p == '{') {
            ++p;
            if (eat('}')) return;
            do {
                (void)str();
                if (!eat(':')) { fail(); return; }
                skip(depth + 1);
            } while (ok && eat(','));
            if (!eat('}')) fail();
            return;
        }
        if (*p == '[') {
            ++p;
            if (eat(']')) return;
            do skip(depth + 1); while (ok && eat(','));
            if (!eat(']')) fail();
            return;
        }
        // number / true / false / null
        const char* q = p;
        while (q < e && *q != ',' && *q != '}' && *q != ']' && *q != ' ' && *q != '\n' && *q != '\r' &&
               *q != '\t')
            ++q;
        if (q == p) fail();
        p = q;
    }
    bool int_array(std::vector<int64_t>& v) {
        if (!eat('[')) return false;
        if (eat(']')) return true;
        do {
            int64_t x;
            if (!integer(&x)) return false;
            v.push_back(x);
        } while (eat(','));
        return eat(']');
    }
};

int32_t dtype_code(const std::string& s) {
    // dtype_from_string, include/servoflow/core/dtype.h:57-66
    if (s == "F32" || s == "float32") return SF_F32;
    if (s == "F16" || s == "float16") return SF_F16;
    if (s == "BF16" || s == "bfloat16") return SF_BF16;
    if (s == "I8" || s == "int8") return SF_I8;
    if (s == "I32" || s == "int32") return SF_I32;
    return -1;
}

size_t dtype_bytes(int32_t dt) {
    switch (dt) {
        case SF_F32: return 4;
        case SF_F16: return 2;
        case SF_BF16: return 2;
        case SF_I8: return 1;
        case SF_I32: return 4;
        default: return 0;
    }
}

bool parse_header(const char* data, size_t size, std::vector<StTensor>& out, uint64_t* data_off,
                  std::string& err) {
    if (size < 8) { err = "file too small"; return false; }
    uint64_t hl = 0;
    std::memcpy(&hl, data, 8);   // little-endian on the hosts this runs on
    if (hl > size - 8) { err = "header length exceeds file size"; return false; }
    *data_off = 8 + hl;
    Json j{data + 8, data + 8 + hl};
    if (!j.eat('{')) { err = "header is not a JSON object"; return false; }
    if (j.eat('}')) return true;
    do {
        std::string key = j.str();
        if (!j.ok || !j.eat(':')) { err = "malformed header"; return false; }
        if (key == "__metadata__") {
            j.skip();
            continue;
        }
        StTensor t;
        t.name = key;
        if (!j.eat('{')) { err = "tensor entry is not an object: " + key; return false; }
        bool have_dt = false, have_shape = false, have_off = false;
        if (!j.eat('}')) {
            do {
                const std::string f = j.str();
                if (!j.ok || !j.eat(':')) { err = "malformed entry: " + key; return false; }
                if (f == "dtype") {
                    t.dtype = dtype_code(j.str());
                    have_dt = j.ok;
                } else if (f == "shape") {
                    have_shape = j.int_array(t.shape);
                } else if (f == "data_offsets") {
                    std::vector<int64_t> o;
                    if (!j.int_array(o) || o.size() != 2 || o[0] < 0 || o[1] < o[0]) {
                        err = "bad data_offsets: " + key;
                        return false;
                    }
                    t.begin = (uint64_t)o[0];
                    t.end = (uint64_t)o[1];
                    have_off = true;
                } else {
                    j.skip();
                }
            } while (j.ok && j.eat(','));
            if (!j.eat('}')) { err = "malformed entry: " + key; return false; }
        }
        if (!have_dt || !have_shape || !have_off) { err = "incomplete entry: " + key; return false; }
        for (int64_t d : t.shape)
            if (d < 0) { err = "negative dim: " + key; return false; }
        out.push_back(std::move(t));
    } while (j.ok && j.eat(','));
    if (!j.ok || !j.eat('}')) { err = "malformed header"; return false; }
    return true;
}

struct Mapped {
    int fd = -1;
    const char* data = nullptr;
    size_t size = 0;
    explicit Mapped(const char* path) {
        fd = ::open(path, O_RDONLY);
        if (fd < 0) return;
        struct stat st{};
        if (::fstat(fd, &st) != 0) return;
        size = (size_t)st.st_size;
        if (size == 0) return;
        void* p = ::mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (p == MAP_FAILED) return;
        data = static_cast<const char*>(p);
        ::madvise(p, size, MADV_SEQUENTIAL);
    }
    ~Mapped() {
        if (data) ::munmap(const_cast<char*>(data), size);
        if (fd >= 0) ::close(fd);
    }
    Mapped(const Mapped&) = delete;
    Mapped& operator=(const Mapped&) = delete;
};

float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1F, man = h & 0x3FF, bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {   // subnormal: renormalise
            int e = -1;
            do { ++e; man <<= 1; } while (!(man & 0x400));
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3FF) << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

uint16_t f32_to_bf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

void to_f32(const char* src, int32_t dt, size_t n, std::vector<float>& out) {
    out.resize(n);
    for (size_t i = 0; i < n; ++i) {
        if (dt == SF_F32) {
            std::memcpy(&out[i], src + 4 * i, 4);
        } else {
            uint16_t h;
            std::memcpy(&h, src + 2 * i, 2);
            if (dt == SF_F16) {
                out[i] = f16_to_f32(h);
            } else {
                const uint32_t u = (uint32_t)h << 16;
                std::memcpy(&out[i], &u, 4);
            }
        }
    }
}

// remap_key (hf_to_servoflow.py:41-65): "" = skip.
std::string remap_key(const std::string& k) {
    if (k.find(".shadow_params") != std::string::npos || k.rfind("ema_model.", 0) == 0) return "";
    if (k.find("optimizer") != std::string::npos || k.find("scheduler") != std::string::npos) return "";
    if (k.rfind("model.", 0) == 0) return k.substr(6);
    return k;
}

// Shapes agree up to leading 1s ([1, S, D] position tables).
bool same_shape(std::vector<int64_t> a, std::vector<int64_t> b) {
    while (a.size() > 1 && a.front() == 1) a.erase(a.begin());
    while (b.size() > 1 && b.front() == 1) b.erase(b.begin());
    return a == b;
}

}  // namespace

extern "C" int sf_safetensors_inspect(const char* path, sf_st_entry* entries, int32_t max_entries,
                                      int32_t* count) {
    if (!path || !count || max_entries < 0 || (max_entries > 0 && !entries)) return SF_EINVAL;
    *count = 0;
    Mapped f(path);
    if (!f.data) return SF_EINVAL;
    std::vector<StTensor> ts;
    uint64_t off = 0;
    std::string err;
    if (!parse_header(f.data, f.size, ts, &off, err)) return SF_EINVAL;
    *count = (int32_t)ts.size();
    for (int32_t i = 0; i < (int32_t)ts.size() && i < max_entries; ++i) {
        sf_st_entry& e = entries[i];
        std::memset(&e, 0, sizeof e);
        std::strncpy(e.name, ts[i].name.c_str(), sizeof e.name - 1);
        e.dtype = ts[i].dtype;
        e.ndim = (int32_t)std::min<size_t>(ts[i].shape.size(), 8);
        for (int32_t d = 0; d < e.ndim; ++d) e.shape[d] = ts[i].shape[d];
        e.data_begin = off + ts[i].begin;
        e.data_end = off + ts[i].end;
    }
    return SF_OK;
}

extern "C" int sf_rdt_load_safetensors(sf_rdt* m, const char* path, int32_t flags, int32_t* loaded) {
    if (!m || !path) return SF_EINVAL;
    if (loaded) *loaded = 0;
    sf_rdt_set_error(m, "");
    Mapped f(path);
    if (!f.data) {
        sf_rdt_set_error(m, std::string("cannot open or map ") + path);
        return SF_EINVAL;
    }
    std::vector<StTensor> ts;
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
    for (const StTensor& t : ts) {
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
