// SafeTensors header parser, element conversions and sf_safetensors_inspect
// (host only).  The loader that copies tensors to the device is in
// safetensors.cpp.  Citations are to the reference's
// src/loader/safetensors.cpp unless named otherwise.
#include "st_format.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>

#include "sf_hip.h"
#include "sf_rdt.h"

namespace sf_amd {
namespace st {
namespace {

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
            const uint64_t d = (uint64_t)(*q - '0');
            if (v > ((1ull << 62) - d) / 10) return false;   // v * 10 + d > 2^62
            v = v * 10 + d;
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

}  // namespace

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

bool parse_header(const char* data, size_t size, std::vector<Tensor>& out, uint64_t* data_off,
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
        Tensor t;
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

Mapped::Mapped(const char* path) {
    fd_ = ::open(path, O_RDONLY);
    if (fd_ < 0) return;
    struct stat sb{};
    if (::fstat(fd_, &sb) != 0 || sb.st_size <= 0) return;
    void* p = ::mmap(nullptr, (size_t)sb.st_size, PROT_READ, MAP_PRIVATE, fd_, 0);
    if (p == MAP_FAILED) return;
    data = static_cast<const char*>(p);
    size = (size_t)sb.st_size;
    ::madvise(p, size, MADV_SEQUENTIAL);
}

Mapped::~Mapped() {
    if (data) ::munmap(const_cast<char*>(data), size);
    if (fd_ >= 0) ::close(fd_);
}

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

}  // namespace st
}  // namespace sf_amd

extern "C" int sf_safetensors_inspect(const char* path, sf_st_entry* entries, int32_t max_entries,
                                      int32_t* count) {
    if (!path || !count || max_entries < 0 || (max_entries > 0 && !entries)) return SF_EINVAL;
    *count = 0;
    sf_amd::st::Mapped f(path);
    if (!f.data) return SF_EINVAL;
    std::vector<sf_amd::st::Tensor> ts;
    uint64_t off = 0;
    std::string err;
    if (!sf_amd::st::parse_header(f.data, f.size, ts, &off, err)) return SF_EINVAL;
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

