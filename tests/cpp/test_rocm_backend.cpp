// Tests of RocmBackend::attention (servoflow_amd/host/rocm_backend.h), the
// IBackend::attention-shaped layer (include/servoflow/backend/backend.h:105-110),
// written in the style of the reference's C++ tests (tests/test_*.cpp): one
// function per case, inputs from a fixed seed, results checked against the
// CPU oracle (oracle/sf_oracle.h, test infrastructure only).
//
// Tolerances as the Python parity tests: fp32 output within max-abs 2e-2 and
// sum|d| / sum|ref| 1e-3 of the fp32 oracle on the same bf16-rounded inputs.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <stdexcept>
#include <string>
#include <vector>

#include "rocm_backend.h"
extern "C" {
#include "sf_oracle.h"
}

using sf_amd::DType;
using sf_amd::RocmBackend;
using sf_amd::TensorRef;

namespace {

int g_failed = 0;

#define CHECK(cond, msg)                                                              \
    do {                                                                              \
        if (!(cond)) throw std::runtime_error(std::string("check failed: ") + (msg)); \
    } while (0)

#define HIP_OK(expr) CHECK((expr) == hipSuccess, #expr)

void run_case(const char* name, const std::function<void()>& fn) {
    try {
        fn();
        std::printf("[ OK   ] %s\n", name);
    } catch (const std::exception& e) {
        std::printf("[ FAIL ] %s: %s\n", name, e.what());
        ++g_failed;
    }
    std::fflush(stdout);
}

uint16_t to_bf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return (uint16_t)(u >> 16);   // inputs are already bf16-rounded: exact
}

struct DevBuf {
    void* p = nullptr;
    size_t n = 0;
    explicit DevBuf(size_t bytes) : n(bytes) {
        if (hipMalloc(&p, bytes) != hipSuccess) throw std::runtime_error("hipMalloc");
    }
    ~DevBuf() { (void)hipFree(p); }
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
};

// N(0,1) from the oracle's generator, rounded to bf16; host fp32 copy + device bf16.
struct Bf16Tensor {
    std::vector<float> host;
    DevBuf dev;
    std::vector<int64_t> shape;
    Bf16Tensor(uint64_t seed, std::vector<int64_t> shp)
        : host(numel(shp)), dev(numel(shp) * 2), shape(shp) {
        sfo_randn(seed, (int64_t)host.size(), 1.f, host.data());
        sfo_bf16_round_array(host.data(), (int64_t)host.size());
        std::vector<uint16_t> b(host.size());
        for (size_t i = 0; i < host.size(); ++i) b[i] = to_bf16(host[i]);
        if (hipMemcpy(dev.p, b.data(), b.size() * 2, hipMemcpyHostToDevice) != hipSuccess)
            throw std::runtime_error("hipMemcpy");
    }
    static size_t numel(const std::vector<int64_t>& s) {
        size_t n = 1;
        for (int64_t x : s) n *= (size_t)x;
        return n;
    }
    TensorRef ref() const { return TensorRef::contiguous(dev.p, DType::BFloat16, shape); }
};

std::vector<float> download_f32(const DevBuf& b, size_t n) {
    std::vector<float> h(n);
    if (hipMemcpy(h.data(), b.p, n * 4, hipMemcpyDeviceToHost) != hipSuccess)
        throw std::runtime_error("hipMemcpy D2H");
    return h;
}

void expect_close(const std::vector<float>& got, const std::vector<float>& ref, const char* what) {
    CHECK(got.size() == ref.size(), what);
    double sd = 0, sr = 0, mx = 0;
    for (size_t i = 0; i < got.size(); ++i) {
        CHECK(std::isfinite(got[i]), what);
        const double d = std::fabs((double)got[i] - ref[i]);
        sd += d;
        sr += std::fabs((double)ref[i]);
        if (d > mx) mx = d;
    }
    const double mr = sr > 0 ? sd / sr : sd;
    if (!(mx <= 2e-2 && mr <= 1e-3)) {
        char buf[160];
        std::snprintf(buf, sizeof buf, "%s: max-abs %.3e mean-rel %.3e", what, mx, mr);
        throw std::runtime_error(buf);
    }
}

// The oracle over a subset of keys of one batch element (key-padding mask).
std::vector<float> oracle_kept(const Bf16Tensor& q, const Bf16Tensor& k, const Bf16Tensor& v,
                               const std::vector<std::vector<uint8_t>>& keep) {
    const int B = (int)q.shape[0], H = (int)q.shape[1], S = (int)q.shape[2], D = (int)q.shape[3];
    const int Sk = (int)k.shape[2];
    std::vector<float> out((size_t)B * H * S * D, 0.f);
    for (int b = 0; b < B; ++b) {
        std::vector<int> idx;
        for (int j = 0; j < Sk; ++j)
            if (keep[b][j]) idx.push_back(j);
        if (idx.empty()) continue;
        const int n = (int)idx.size();
        std::vector<float> kk((size_t)H * n * D), vv((size_t)H * n * D), o((size_t)H * S * D);
        for (int h = 0; h < H; ++h)
            for (int j = 0; j < n; ++j)
                for (int d = 0; d < D; ++d) {
                    const size_t src = (((size_t)b * H + h) * Sk + idx[j]) * D + d;
                    kk[((size_t)h * n + j) * D + d] = k.host[src];
                    vv[((size_t)h * n + j) * D + d] = v.host[src];
                }
        sfo_attention_f32(q.host.data() + (size_t)b * H * S * D, kk.data(), vv.data(), o.data(), 1, H,
                          S, n, D, 0.f, 0, nullptr);
        std::memcpy(out.data() + (size_t)b * H * S * D, o.data(), o.size() * 4);
    }
    return out;
}

void test_self_attention_matches_oracle() {
    RocmBackend be;
    Bf16Tensor q(11, {1, 32, 67, 64}), k(12, {1, 32, 67, 64}), v(13, {1, 32, 67, 64});
    DevBuf ob((size_t)32 * 67 * 64 * 4);
    TensorRef out = TensorRef::contiguous(ob.p, DType::Float32, {1, 32, 67, 64});
    be.attention(q.ref(), k.ref(), v.ref(), out);
    HIP_OK(hipDeviceSynchronize());
    std::vector<float> ref(q.host.size());
    sfo_attention_f32(q.host.data(), k.host.data(), v.host.data(), ref.data(), 1, 32, 67, 67, 64, 0.f,
                      0, nullptr);
    expect_close(download_f32(ob, ref.size()), ref, "self 1x32x67x67");
}

void test_int32_mask_is_valid_lengths() {
    RocmBackend be;
    const int B = 2, H = 4, S = 67, Sk = 4374;
    Bf16Tensor q(21, {B, H, S, 64}), k(22, {B, H, Sk, 64}), v(23, {B, H, Sk, 64});
    const int32_t lens[B] = {4000, 517};
    DevBuf lb(sizeof lens);
    HIP_OK(hipMemcpy(lb.p, lens, sizeof lens, hipMemcpyHostToDevice));
    TensorRef mask = TensorRef::contiguous(lb.p, DType::Int32, {B});
    DevBuf ob((size_t)B * H * S * 64 * 4);
    TensorRef out = TensorRef::contiguous(ob.p, DType::Float32, {B, H, S, 64});
    be.attention(q.ref(), k.ref(), v.ref(), out, &mask);
    HIP_OK(hipDeviceSynchronize());
    std::vector<float> ref(q.host.size());
    sfo_attention_f32(q.host.data(), k.host.data(), v.host.data(), ref.data(), B, H, S, Sk, 64, 0.f, 0,
                      lens);
    expect_close(download_f32(ob, ref.size()), ref, "Int32 lengths");
}

void test_bool_key_padding_mask_both_shapes() {
    RocmBackend be;
    const int B = 2, H = 2, S = 67, Sk = 300, pitch = 300;
    Bf16Tensor q(31, {B, H, S, 64}), k(32, {B, H, Sk, 64}), v(33, {B, H, Sk, 64});
    std::vector<std::vector<uint8_t>> keep(B, std::vector<uint8_t>(pitch, 0));
    std::vector<float> u(B * Sk);
    sfo_randn(34, (int64_t)u.size(), 1.f, u.data());
    for (int b = 0; b < B; ++b)
        for (int j = 0; j < Sk; ++j) keep[b][j] = u[b * Sk + j] > -0.3f ? 1 : 0;
    DevBuf mb((size_t)B * pitch);
    for (int b = 0; b < B; ++b)
        HIP_OK(hipMemcpy(static_cast<char*>(mb.p) + b * pitch, keep[b].data(), pitch, hipMemcpyHostToDevice));
    const std::vector<float> ref = oracle_kept(q, k, v, keep);
    for (int form = 0; form < 2; ++form) {
        TensorRef mask = form == 0 ? TensorRef::contiguous(mb.p, DType::Bool, {B, Sk})
                                   : TensorRef::contiguous(mb.p, DType::Bool, {B, 1, 1, Sk});
        DevBuf ob((size_t)B * H * S * 64 * 4);
        TensorRef out = TensorRef::contiguous(ob.p, DType::Float32, {B, H, S, 64});
        be.attention(q.ref(), k.ref(), v.ref(), out, &mask);
        HIP_OK(hipDeviceSynchronize());
        expect_close(download_f32(ob, ref.size()), ref, form == 0 ? "Bool [B,Sk]" : "Bool [B,1,1,Sk]");
    }
}

void test_strided_output_and_explicit_scale() {
    RocmBackend be;
    const int B = 1, H = 8, S = 67, Sk = 1024;
    Bf16Tensor q(41, {B, H, S, 64}), k(42, {B, H, Sk, 64}), v(43, {B, H, Sk, 64});
    // out as a [B, S, H, D] buffer viewed as [B, H, S, D] (the block's layout)
    DevBuf ob((size_t)B * S * H * 64 * 4);
    TensorRef out;
    out.data = ob.p;
    out.dtype = DType::Float32;
    out.shape = {B, H, S, 64};
    out.strides = {(int64_t)S * H * 64 * 4, 64 * 4, (int64_t)H * 64 * 4, 4};
    out.on_device = true;
    be.attention(q.ref(), k.ref(), v.ref(), out, nullptr, 0.3f);
    HIP_OK(hipDeviceSynchronize());
    std::vector<float> ref(q.host.size());
    sfo_attention_f32(q.host.data(), k.host.data(), v.host.data(), ref.data(), B, H, S, Sk, 64, 0.3f, 0,
                      nullptr);
    std::vector<float> seq = download_f32(ob, ref.size()), got(ref.size());
    for (int h = 0; h < H; ++h)
        for (int s = 0; s < S; ++s)
            for (int d = 0; d < 64; ++d)
                got[((size_t)h * S + s) * 64 + d] = seq[((size_t)s * H + h) * 64 + d];
    expect_close(got, ref, "BSHD view, scale 0.3");
}

void test_causal() {
    RocmBackend be;
    Bf16Tensor q(51, {1, 4, 67, 64}), k(52, {1, 4, 67, 64}), v(53, {1, 4, 67, 64});
    DevBuf ob((size_t)4 * 67 * 64 * 4);
    TensorRef out = TensorRef::contiguous(ob.p, DType::Float32, {1, 4, 67, 64});
    be.attention(q.ref(), k.ref(), v.ref(), out, nullptr, 0.f, true);
    HIP_OK(hipDeviceSynchronize());
    std::vector<float> ref(q.host.size());
    sfo_attention_f32(q.host.data(), k.host.data(), v.host.data(), ref.data(), 1, 4, 67, 67, 64, 0.f, 1,
                      nullptr);
    expect_close(download_f32(ob, ref.size()), ref, "causal");
}

template <class E>
void expect_throw(const std::function<void()>& fn, const char* what) {
    try {
        fn();
    } catch (const E&) {
        return;
    } catch (const std::exception& e) {
        throw std::runtime_error(std::string(what) + ": wrong exception type: " + e.what());
    }
    throw std::runtime_error(std::string(what) + ": no exception");
}

void test_errors_use_reference_exception_types() {
    RocmBackend be;
    Bf16Tensor q(61, {1, 2, 8, 64}), k(62, {1, 2, 300, 64});
    DevBuf ob((size_t)2 * 8 * 64 * 4);
    TensorRef out = TensorRef::contiguous(ob.p, DType::Float32, {1, 2, 8, 64});
    TensorRef qf = q.ref();
    qf.dtype = DType::Float32;   // wrong dtype
    expect_throw<std::invalid_argument>([&] { be.attention(qf, k.ref(), k.ref(), out); }, "fp32 inputs");
    TensorRef qh = q.ref();
    qh.on_device = false;        // host tensor (cuda_backend.cu:156-161)
    expect_throw<std::invalid_argument>([&] { be.attention(qh, k.ref(), k.ref(), out); }, "host tensor");
    DevBuf fm((size_t)8 * 300 * 4);
    TensorRef additive = TensorRef::contiguous(fm.p, DType::Float32, {1, 1, 8, 299});
    expect_throw<std::invalid_argument>([&] { be.attention(q.ref(), k.ref(), k.ref(), out, &additive); },
                                        "additive float mask of the wrong shape");
    DevBuf bm((size_t)8 * 300);
    TensorRef per_query = TensorRef::contiguous(bm.p, DType::Bool, {1, 1, 8, 300});
    expect_throw<std::invalid_argument>([&] { be.attention(q.ref(), k.ref(), k.ref(), out, &per_query); },
                                        "per-query Bool mask");
    Bf16Tensor q128(63, {1, 1, 4, 128});
    DevBuf ob128((size_t)4 * 128 * 4);
    TensorRef out128 = TensorRef::contiguous(ob128.p, DType::Float32, {1, 1, 4, 128});
    expect_throw<std::invalid_argument>([&] { be.attention(q128.ref(), q128.ref(), q128.ref(), out128); },
                                        "head dim 128");
    TensorRef bad_shape = k.ref();
    bad_shape.shape[3] = 32;
    expect_throw<std::invalid_argument>([&] { be.attention(q.ref(), bad_shape, k.ref(), out); }, "shape mismatch");
}

void test_graph_capture_with_reserved_workspace() {
    const int B = 1, H = 32, S = 67, Sk = 4374;
    Bf16Tensor q(71, {B, H, S, 64}), k(72, {B, H, Sk, 64}), v(73, {B, H, Sk, 64});
    DevBuf ob((size_t)B * H * S * 64 * 4), eb((size_t)B * H * S * 64 * 4);
    TensorRef out = TensorRef::contiguous(ob.p, DType::Float32, {B, H, S, 64});
    TensorRef eager = TensorRef::contiguous(eb.p, DType::Float32, {B, H, S, 64});
    hipStream_t st;
    HIP_OK(hipStreamCreate(&st));
    {
        // capture without a reserved workspace: refused with runtime_error
        RocmBackend fresh;
        HIP_OK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        bool threw = false;
        try {
            fresh.attention(q.ref(), k.ref(), v.ref(), out, nullptr, 0.f, false, st);
        } catch (const std::runtime_error&) {
            threw = true;
        }
        hipGraph_t g0 = nullptr;
        (void)hipStreamEndCapture(st, &g0);
        if (g0) (void)hipGraphDestroy(g0);
        CHECK(threw, "capture without reserve must throw std::runtime_error");
    }
    RocmBackend be;
    be.reserve_attention_workspace(RocmBackend::attention_workspace_bytes(q.ref(), k.ref()), st);
    be.attention(q.ref(), k.ref(), v.ref(), eager, nullptr, 0.f, false, st);
    HIP_OK(hipStreamSynchronize(st));
    hipGraph_t g;
    hipGraphExec_t ge;
    HIP_OK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    be.attention(q.ref(), k.ref(), v.ref(), out, nullptr, 0.f, false, st);
    HIP_OK(hipStreamEndCapture(st, &g));
    HIP_OK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
    const std::vector<float> ref = download_f32(eb, (size_t)B * H * S * 64);
    for (int rep = 0; rep < 3; ++rep) {
        HIP_OK(hipMemsetAsync(ob.p, 0xff, ob.n, st));   // NaN fill, outside the graph
        HIP_OK(hipGraphLaunch(ge, st));
        HIP_OK(hipStreamSynchronize(st));
        const std::vector<float> got = download_f32(ob, ref.size());
        CHECK(std::memcmp(got.data(), ref.data(), ref.size() * 4) == 0, "graph replay == eager");
    }
    (void)hipGraphExecDestroy(ge);
    (void)hipGraphDestroy(g);
    (void)hipStreamDestroy(st);
}

// A tensor of any input dtype: N(0,1) rounded to that dtype on the host
// (fp32 copy for the oracle), stored on the device in that dtype.
struct AnyTensor {
    std::vector<float> host;
    DevBuf dev;
    std::vector<int64_t> shape;
    DType dt;
    AnyTensor(uint64_t seed, std::vector<int64_t> shp, DType t)
        : host(Bf16Tensor::numel(shp)), dev(Bf16Tensor::numel(shp) * sf_amd::dtype_size(t)), shape(shp), dt(t) {
        sfo_randn(seed, (int64_t)host.size(), 1.f, host.data());
        std::vector<uint16_t> h16(host.size());
        for (size_t i = 0; i < host.size(); ++i) {
            if (t == DType::Float16) {
                const _Float16 x = (_Float16)host[i];
                host[i] = (float)x;
                std::memcpy(&h16[i], &x, 2);
            } else if (t == DType::BFloat16) {
                host[i] = sfo_bf16_round(host[i]);
                h16[i] = to_bf16(host[i]);
            }
        }
        const void* src = t == DType::Float32 ? static_cast<const void*>(host.data()) : h16.data();
        if (hipMemcpy(dev.p, src, dev.n, hipMemcpyHostToDevice) != hipSuccess) throw std::runtime_error("hipMemcpy");
    }
    TensorRef ref() const { return TensorRef::contiguous(dev.p, dt, shape); }
};

// fp32 output of RocmBackend::attention for one input dtype vs the oracle.
void dtype_case(DType dt, int B, int H, int S, int Sk, const int32_t* lens, double max_abs, double mean_rel,
                const char* what) {
    RocmBackend be;
    AnyTensor q(81 + Sk, {B, H, S, 64}, dt), k(82 + Sk, {B, H, Sk, 64}, dt), v(83 + Sk, {B, H, Sk, 64}, dt);
    DevBuf ob((size_t)B * H * S * 64 * 4);
    TensorRef out = TensorRef::contiguous(ob.p, DType::Float32, {B, H, S, 64});
    DevBuf lb(lens ? (size_t)B * 4 : 4);
    TensorRef mask;
    if (lens) {
        HIP_OK(hipMemcpy(lb.p, lens, (size_t)B * 4, hipMemcpyHostToDevice));
        mask = TensorRef::contiguous(lb.p, DType::Int32, {B});
    }
    be.attention(q.ref(), k.ref(), v.ref(), out, lens ? &mask : nullptr);
    HIP_OK(hipDeviceSynchronize());
    std::vector<float> ref(q.host.size());
    sfo_attention_f32(q.host.data(), k.host.data(), v.host.data(), ref.data(), B, H, S, Sk, 64, 0.f, 0, lens);
    const std::vector<float> got = download_f32(ob, ref.size());
    double sd = 0, sr = 0, mx = 0;
    for (size_t i = 0; i < got.size(); ++i) {
        CHECK(std::isfinite(got[i]), what);
        const double d = std::fabs((double)got[i] - ref[i]);
        sd += d;
        sr += std::fabs((double)ref[i]);
        mx = d > mx ? d : mx;
    }
    if (!(mx <= max_abs && sd / sr <= mean_rel)) {
        char buf[200];
        std::snprintf(buf, sizeof buf, "%s: max-abs %.3e mean-rel %.3e", what, mx, sd / sr);
        throw std::runtime_error(buf);
    }
}

void test_float16_tensors() {
    // the reference's default compute dtype (config.h:57); exact P.V form
    dtype_case(DType::Float16, 1, 32, 67, 67, nullptr, 2e-2, 2e-5, "Float16 self 1x32x67x67");
    dtype_case(DType::Float16, 1, 32, 67, 4374, nullptr, 2e-2, 2e-5, "Float16 image 1x32x67x4374");
    const int32_t lens[2] = {1024, 333};
    dtype_case(DType::Float16, 2, 32, 67, 1024, lens, 2e-2, 2e-5, "Float16 language, valid lengths");
}

void test_float32_tensors() {
    // the reference's fp32 path (naive kernel, attention.cu:90-139)
    dtype_case(DType::Float32, 1, 32, 67, 67, nullptr, 1e-4, 1e-5, "Float32 self 1x32x67x67");
    const int32_t lens[2] = {700, 32};
    dtype_case(DType::Float32, 2, 32, 67, 1024, lens, 1e-4, 1e-5, "Float32 language, valid lengths");
    dtype_case(DType::Float32, 1, 32, 67, 4374, nullptr, 1e-4, 1e-5, "Float32 image 1x32x67x4374");
}

void test_float16_output() {
    RocmBackend be;
    AnyTensor q(91, {1, 8, 67, 64}, DType::Float16), k(92, {1, 8, 900, 64}, DType::Float16),
        v(93, {1, 8, 900, 64}, DType::Float16);
    DevBuf o16((size_t)8 * 67 * 64 * 2), o32((size_t)8 * 67 * 64 * 4);
    TensorRef out16 = TensorRef::contiguous(o16.p, DType::Float16, {1, 8, 67, 64});
    TensorRef out32 = TensorRef::contiguous(o32.p, DType::Float32, {1, 8, 67, 64});
    be.attention(q.ref(), k.ref(), v.ref(), out16);
    be.attention(q.ref(), k.ref(), v.ref(), out32);
    HIP_OK(hipDeviceSynchronize());
    const size_t n = (size_t)8 * 67 * 64;
    std::vector<uint16_t> h16(n);
    HIP_OK(hipMemcpy(h16.data(), o16.p, n * 2, hipMemcpyDeviceToHost));
    const std::vector<float> f32 = download_f32(o32, n);
    for (size_t i = 0; i < n; ++i) {
        _Float16 x;
        std::memcpy(&x, &h16[i], 2);
        const double ulp = std::fabs(f32[i]) * std::ldexp(1.0, -10) + std::ldexp(1.0, -24);
        CHECK(std::fabs((double)(float)x - f32[i]) <= ulp, "Float16 out = fp32 out rounded");
    }
}

void test_streams_have_separate_workspaces() {
    // two image cross-attentions (7 key splits each, so both need partials)
    // queued on two streams before either is waited for
    const int B = 1, H = 32, S = 67, Sk = 4374;
    Bf16Tensor q1(101, {B, H, S, 64}), k1(102, {B, H, Sk, 64}), v1(103, {B, H, Sk, 64});
    Bf16Tensor q2(104, {B, H, S, 64}), k2(105, {B, H, Sk, 64}), v2(106, {B, H, Sk, 64});
    DevBuf o1((size_t)B * H * S * 64 * 4), o2((size_t)B * H * S * 64 * 4);
    TensorRef out1 = TensorRef::contiguous(o1.p, DType::Float32, {B, H, S, 64});
    TensorRef out2 = TensorRef::contiguous(o2.p, DType::Float32, {B, H, S, 64});
    hipStream_t s1, s2;
    HIP_OK(hipStreamCreate(&s1));
    HIP_OK(hipStreamCreate(&s2));
    RocmBackend be;
    for (int rep = 0; rep < 4; ++rep) {
        be.attention(q1.ref(), k1.ref(), v1.ref(), out1, nullptr, 0.f, false, s1);
        be.attention(q2.ref(), k2.ref(), v2.ref(), out2, nullptr, 0.f, false, s2);
    }
    HIP_OK(hipStreamSynchronize(s1));
    HIP_OK(hipStreamSynchronize(s2));
    std::vector<float> r1(q1.host.size()), r2(q2.host.size());
    sfo_attention_f32(q1.host.data(), k1.host.data(), v1.host.data(), r1.data(), B, H, S, Sk, 64, 0.f, 0, nullptr);
    sfo_attention_f32(q2.host.data(), k2.host.data(), v2.host.data(), r2.data(), B, H, S, Sk, 64, 0.f, 0, nullptr);
    expect_close(download_f32(o1, r1.size()), r1, "stream 1");
    expect_close(download_f32(o2, r2.size()), r2, "stream 2");
    (void)hipStreamDestroy(s1);
    (void)hipStreamDestroy(s2);
}

void test_precision_option_and_large_v() {
    // a V element of 2^17 (finite in bf16): the default (exact) precision
    // returns finite values matching the oracle; the fast form documents
    // inf/NaN in that head dim's column
    const int B = 1, H = 2, S = 67, Sk = 600;
    Bf16Tensor q(111, {B, H, S, 64}), k(112, {B, H, Sk, 64}), v(113, {B, H, Sk, 64});
    const size_t big = ((size_t)0 * Sk + 17) * 64 + 5;   // head 0, key 17, dim 5
    v.host[big] = 131072.f;
    const uint16_t bits = to_bf16(131072.f);
    HIP_OK(hipMemcpy(static_cast<uint16_t*>(v.dev.p) + big, &bits, 2, hipMemcpyHostToDevice));
    DevBuf ob((size_t)B * H * S * 64 * 4);
    TensorRef out = TensorRef::contiguous(ob.p, DType::Float32, {B, H, S, 64});
    RocmBackend exact;
    CHECK(exact.precision() == sf_amd::AttentionPrecision::Exact, "default precision is exact");
    exact.attention(q.ref(), k.ref(), v.ref(), out);
    HIP_OK(hipDeviceSynchronize());
    std::vector<float> ref(q.host.size());
    sfo_attention_f32(q.host.data(), k.host.data(), v.host.data(), ref.data(), B, H, S, Sk, 64, 0.f, 0, nullptr);
    const std::vector<float> got = download_f32(ob, ref.size());
    double sd = 0, sr = 0;
    for (size_t i = 0; i < got.size(); ++i) {
        CHECK(std::isfinite(got[i]), "exact precision: finite output for large V");
        sd += std::fabs((double)got[i] - ref[i]);
        sr += std::fabs((double)ref[i]);
    }
    CHECK(sd / sr <= 1e-4, "exact precision matches the oracle with large V");
    RocmBackend fast(sf_amd::AttentionPrecision::Fast);
    fast.attention(q.ref(), k.ref(), v.ref(), out);
    HIP_OK(hipDeviceSynchronize());
    const std::vector<float> gf = download_f32(ob, ref.size());
    bool col_nonfinite = false;
    for (int s = 0; s < S; ++s) col_nonfinite |= !std::isfinite(gf[(size_t)s * 64 + 5]);
    CHECK(col_nonfinite, "fast precision: |v| >= 2^16 reaches its column as inf/NaN");
    for (size_t i = 0; i < gf.size(); ++i)
        if (i % 64 != 5) CHECK(std::isfinite(gf[i]), "fast precision: other columns finite");
}

// Uploads a float host mask [rows][Sk] (rows = B or B*S) to the device.
struct FloatMask {
    DevBuf dev;
    std::vector<int64_t> shape;
    FloatMask(const std::vector<float>& h, std::vector<int64_t> shp) : dev(h.size() * 4), shape(shp) {
        if (hipMemcpy(dev.p, h.data(), h.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
            throw std::runtime_error("hipMemcpy");
    }
    TensorRef ref() const { return TensorRef::contiguous(dev.p, DType::Float32, shape); }
};

void test_additive_mask_forms() {
    // the additive mask of backend.h:104 (softmax(Q K^T scale + mask)):
    // 0 / -1e4 / -inf per key, a row offset by a constant, and a row that is
    // all -1e4 (the additive form then keeps every key: the offset cancels)
    const int B = 3, H = 4, S = 20, Sk = 300;
    Bf16Tensor q(301, {B, H, S, 64}), k(302, {B, H, Sk, 64}), v(303, {B, H, Sk, 64});
    std::vector<float> m((size_t)B * Sk);
    std::vector<std::vector<uint8_t>> keep(B, std::vector<uint8_t>(Sk));
    for (int j = 0; j < Sk; ++j) {
        const bool k0 = (j * 7) % 5 != 0;
        m[j] = k0 ? 0.f : (j % 2 ? -1e4f : -INFINITY);
        keep[0][j] = k0;
        const bool k1 = j < 123;
        m[Sk + j] = k1 ? 2.5f : -2e4f;   // kept keys share an offset of 2.5
        keep[1][j] = k1;
        m[2 * Sk + j] = -1e4f;
        keep[2][j] = 1;
    }
    const std::vector<float> ref = oracle_kept(q, k, v, keep);
    RocmBackend be;
    DevBuf ob((size_t)B * H * S * 64 * 4), ob2((size_t)B * H * S * 64 * 4);
    TensorRef out = TensorRef::contiguous(ob.p, DType::Float32, {B, H, S, 64});
    TensorRef out2 = TensorRef::contiguous(ob2.p, DType::Float32, {B, H, S, 64});
    FloatMask key_only(m, {B, 1, 1, Sk});
    TensorRef km = key_only.ref();
    be.attention(q.ref(), k.ref(), v.ref(), out, &km);
    HIP_OK(hipDeviceSynchronize());
    const std::vector<float> got = download_f32(ob, ref.size());
    expect_close(got, ref, "additive [B,1,1,Sk] vs oracle on the kept keys");
    // the per-query form with identical rows: the same result bit for bit
    std::vector<float> mq((size_t)B * S * Sk);
    for (int b = 0; b < B; ++b)
        for (int r = 0; r < S; ++r) std::memcpy(&mq[((size_t)b * S + r) * Sk], &m[(size_t)b * Sk], Sk * 4);
    FloatMask per_query(mq, {B, 1, S, Sk});
    TensorRef pq = per_query.ref();
    be.attention(q.ref(), k.ref(), v.ref(), out2, &pq);
    HIP_OK(hipDeviceSynchronize());
    CHECK(std::memcmp(download_f32(ob2, ref.size()).data(), got.data(), got.size() * 4) == 0,
          "additive [B,1,S,Sk] with equal rows == [B,1,1,Sk]");
    // a bfloat16 mask of the same values
    std::vector<uint16_t> mb(m.size());
    for (size_t i = 0; i < m.size(); ++i) {
        uint32_t u;
        std::memcpy(&u, &m[i], 4);
        mb[i] = (uint16_t)(u >> 16);   // 0, -9984 (-1e4 truncated), -2e4, 2.5, -inf: kept / >= 5000 below
    }
    DevBuf bm(mb.size() * 2);
    HIP_OK(hipMemcpy(bm.p, mb.data(), mb.size() * 2, hipMemcpyHostToDevice));
    TensorRef bmask = TensorRef::contiguous(bm.p, DType::BFloat16, {B, 1, 1, Sk});
    be.attention(q.ref(), k.ref(), v.ref(), out2, &bmask);
    HIP_OK(hipDeviceSynchronize());
    CHECK(std::memcmp(download_f32(ob2, ref.size()).data(), got.data(), got.size() * 4) == 0,
          "BFloat16 additive mask == Float32");
    // no key-padding form: a bias between -5000 and the maximum, rows that
    // differ per query, NaN
    std::vector<float> bias = m;
    bias[5] = -0.5f;
    FloatMask fb(bias, {B, 1, 1, Sk});
    TensorRef fbr = fb.ref();
    expect_throw<std::invalid_argument>([&] { be.attention(q.ref(), k.ref(), v.ref(), out, &fbr); }, "-0.5 bias");
    std::vector<float> mq2 = mq;
    mq2[(size_t)(1 * S + 3) * Sk + 7] = -1e4f;
    FloatMask fq(mq2, {B, 1, S, Sk});
    TensorRef fqr = fq.ref();
    expect_throw<std::invalid_argument>([&] { be.attention(q.ref(), k.ref(), v.ref(), out, &fqr); },
                                        "rows differing per query");
    std::vector<float> nan = m;
    nan[9] = NAN;
    FloatMask fn(nan, {B, 1, 1, Sk});
    TensorRef fnr = fn.ref();
    expect_throw<std::invalid_argument>([&] { be.attention(q.ref(), k.ref(), v.ref(), out, &fnr); }, "NaN entry");
    // read on the host: refused inside a graph capture
    hipStream_t st;
    HIP_OK(hipStreamCreate(&st));
    be.reserve_attention_workspace(RocmBackend::attention_workspace_bytes(q.ref(), k.ref()), st);
    HIP_OK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    bool threw = false;
    try {
        be.attention(q.ref(), k.ref(), v.ref(), out, &km, 0.f, false, st);
    } catch (const std::invalid_argument&) {
        threw = true;
    }
    hipGraph_t g0 = nullptr;
    (void)hipStreamEndCapture(st, &g0);
    if (g0) (void)hipGraphDestroy(g0);
    (void)hipStreamDestroy(st);
    CHECK(threw, "additive mask under capture must throw std::invalid_argument");
}

void test_fp32_reserve_then_capture() {
    // the documented flow with no eager call first: reserve the size
    // attention_workspace_bytes() gives for Float32 inputs whose 729 keys
    // take key splits (16-bit inputs would run unsplit), then capture
    const int B = 1, H = 32, S = 67, Sk = 729;
    AnyTensor q(311, {B, H, S, 64}, DType::Float32), k(312, {B, H, Sk, 64}, DType::Float32),
        v(313, {B, H, Sk, 64}, DType::Float32);
    CHECK(RocmBackend::attention_workspace_bytes(q.ref(), k.ref()) > 0, "Float32 729 keys need partials");
    DevBuf ob((size_t)B * H * S * 64 * 4), eb((size_t)B * H * S * 64 * 4);
    TensorRef out = TensorRef::contiguous(ob.p, DType::Float32, {B, H, S, 64});
    TensorRef eager = TensorRef::contiguous(eb.p, DType::Float32, {B, H, S, 64});
    hipStream_t st;
    HIP_OK(hipStreamCreate(&st));
    RocmBackend be;
    be.reserve_attention_workspace(RocmBackend::attention_workspace_bytes(q.ref(), k.ref()), st);
    hipGraph_t g;
    hipGraphExec_t ge;
    HIP_OK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    be.attention(q.ref(), k.ref(), v.ref(), out, nullptr, 0.f, false, st);
    HIP_OK(hipStreamEndCapture(st, &g));
    HIP_OK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
    be.attention(q.ref(), k.ref(), v.ref(), eager, nullptr, 0.f, false, st);
    HIP_OK(hipStreamSynchronize(st));
    const std::vector<float> ref = download_f32(eb, (size_t)B * H * S * 64);
    for (int rep = 0; rep < 2; ++rep) {
        HIP_OK(hipMemsetAsync(ob.p, 0xff, ob.n, st));   // NaN fill, outside the graph
        HIP_OK(hipGraphLaunch(ge, st));
        HIP_OK(hipStreamSynchronize(st));
        CHECK(std::memcmp(download_f32(ob, ref.size()).data(), ref.data(), ref.size() * 4) == 0,
              "Float32 graph replay == eager");
    }
    std::vector<float> oref(ref.size());
    sfo_attention_f32(q.host.data(), k.host.data(), v.host.data(), oref.data(), B, H, S, Sk, 64, 0.f, 0, nullptr);
    expect_close(ref, oref, "Float32 729 keys vs oracle");
    (void)hipGraphExecDestroy(ge);
    (void)hipGraphDestroy(g);
    (void)hipStreamDestroy(st);
}

}  // namespace

int main() {
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) {
        std::printf("no HIP device\n");
        return 2;
    }
    run_case("self_attention_matches_oracle", test_self_attention_matches_oracle);
    run_case("int32_mask_is_valid_lengths", test_int32_mask_is_valid_lengths);
    run_case("bool_key_padding_mask_both_shapes", test_bool_key_padding_mask_both_shapes);
    run_case("strided_output_and_explicit_scale", test_strided_output_and_explicit_scale);
    run_case("causal", test_causal);
    run_case("errors_use_reference_exception_types", test_errors_use_reference_exception_types);
    run_case("graph_capture_with_reserved_workspace", test_graph_capture_with_reserved_workspace);
    run_case("float16_tensors", test_float16_tensors);
    run_case("float32_tensors", test_float32_tensors);
    run_case("float16_output", test_float16_output);
    run_case("streams_have_separate_workspaces", test_streams_have_separate_workspaces);
    run_case("precision_option_and_large_v", test_precision_option_and_large_v);
    run_case("additive_mask_forms", test_additive_mask_forms);
    run_case("fp32_reserve_then_capture", test_fp32_reserve_then_capture);
    if (g_failed) {
        std::printf("%d case(s) failed\n", g_failed);
        return 1;
    }
    std::printf("ALL PASSED\n");
    return 0;
}
