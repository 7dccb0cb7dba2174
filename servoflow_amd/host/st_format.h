// SafeTensors file format: header parsing and element conversions, host
// only (no HIP).  Shared by the checkpoint loader (safetensors.cpp) and the
// host sanitizer build of the tests.
//
// Format (SafeTensorsLoader::parse_header, src/loader/safetensors.cpp:62-108):
// 8-byte little-endian header length, a JSON object {name: {dtype, shape,
// data_offsets}} with an optional "__metadata__" entry, then the data
// section; data_offsets are relative to the end of the header.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace sf_amd {
namespace st {

struct Tensor {
    std::string name;
    int32_t dtype = -1;   // SF_F32 / SF_F16 / SF_BF16 / SF_I8 / SF_I32, -1 unknown
    std::vector<int64_t> shape;
    uint64_t begin = 0, end = 0;   // data_offsets, relative to the data section
};

// dtype_from_string (include/servoflow/core/dtype.h:57-66); -1 when unknown.
int32_t dtype_code(const std::string& s);
// Element size of an SF_* dtype code, 0 when unknown.
size_t dtype_bytes(int32_t dt);

// Parses the 8-byte length and the JSON header of `data[0, size)`.  On
// success fills `out` and `*data_off` (byte offset of the data section).  On
// a malformed or truncated header returns false with a reason in `err`;
// never reads outside `data[0, size)`.  Integers above 2^62, JSON nesting
// deeper than 64 levels and negative dims are header errors.
bool parse_header(const char* data, size_t size, std::vector<Tensor>& out, uint64_t* data_off,
                  std::string& err);

// Read-only memory map of a whole file (data == nullptr when it cannot be
// opened, is empty, or mmap fails).
class Mapped {
public:
    explicit Mapped(const char* path);
    ~Mapped();
    Mapped(const Mapped&) = delete;
    Mapped& operator=(const Mapped&) = delete;
    const char* data = nullptr;
    size_t size = 0;

private:
    int fd_ = -1;
};

// IEEE binary16 -> binary32, exact (subnormals, infinities and NaN kept).
float f16_to_f32(uint16_t h);
// binary32 -> bfloat16, round to nearest even; NaN stays a quiet NaN.
uint16_t f32_to_bf16(float f);
// n elements of an F32 / F16 / BF16 array (unaligned source) into `out`.
void to_f32(const char* src, int32_t dt, size_t n, std::vector<float>& out);
// remap_key (tools/convert/hf_to_servoflow.py:41-65): a leading "model." is
// dropped; EMA, optimizer and scheduler entries map to "" (skipped).
std::string remap_key(const std::string& k);
// Shapes agree up to leading 1s ([1, S, D] position tables vs [S, D]).
bool same_shape(std::vector<int64_t> a, std::vector<int64_t> b);

}  // namespace st
}  // namespace sf_amd
