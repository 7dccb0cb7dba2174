// Host sanitizer run: AddressSanitizer + UndefinedBehaviorSanitizer over the
// CPU code that parses untrusted input or does raw index arithmetic:
//   * the safetensors header parser and sf_safetensors_inspect
//     (servoflow_amd/host/st_format.cpp): a valid header, every truncation,
//     byte substitutions and deletions at every header position, seeded
//     random mutations, deep nesting, integer overflow, hostile lengths;
//   * the element conversions of the checkpoint loader (all 65536 fp16
//     codes against ldexp, bf16 rounding, unaligned sources);
//   * every function of the CPU oracle (oracle/sf_oracle.c) on small ragged
//     shapes, including empty key sets, clamped valid lengths, one-column
//     rows and all-zero int8 rows.
// Built by `make -C tests/cpp sanitize` with g++/gcc -fsanitize=address,
// undefined -fno-sanitize-recover=all: any out-of-bounds access, leak,
// use-after-free, signed overflow or misaligned access aborts with a report.
// Functional checks failing print "FAIL ..." and exit 1.  Host only.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include <unistd.h>

#include "sf_oracle.h"
#include "sf_rdt.h"
#include "st_format.h"

namespace st = sf_amd::st;

static int g_fail = 0;
#define CHECK(cond, ...)                                       \
    do {                                                       \
        if (!(cond)) {                                         \
            std::printf("FAIL %s:%d: ", __FILE__, __LINE__);   \
            std::printf(__VA_ARGS__);                          \
            std::printf("\n");                                 \
            ++g_fail;                                          \
        }                                                      \
    } while (0)

static uint64_t g_rng = 0x5eed5eedULL;
static uint64_t next_u64() {   // xorshift64*
    g_rng ^= g_rng >> 12;
    g_rng ^= g_rng << 25;
    g_rng ^= g_rng >> 27;
    return g_rng * 0x2545F4914F6CDD1DULL;
}

// File image: 8-byte little-endian header length, header, data.
static std::string file_image(const std::string& header, size_t data_bytes) {
    std::string f(8, '\0');
    uint64_t hl = header.size();
    std::memcpy(&f[0], &hl, 8);
    f += header;
    for (size_t i = 0; i < data_bytes; ++i) f += (char)(i * 7 + 1);
    return f;
}

// Parses a copy held in an exact-size heap block, so a read one byte past
// the end is an AddressSanitizer report.
static bool parse_exact(const std::string& img, std::vector<st::Tensor>& out, uint64_t* off,
                        std::string& err) {
    char* buf = static_cast<char*>(std::malloc(img.size() ? img.size() : 1));
    if (!img.empty()) std::memcpy(buf, img.data(), img.size());
    out.clear();
    const bool ok = st::parse_header(buf, img.size(), out, off, err);
    std::free(buf);
    return ok;
}

static const char* kHeader =
    "{\"__metadata__\":{\"format\":\"pt\",\"nested\":[1,[2.5e3,{\"a\":null,\"b\":true}],"
    "\"x\\u00e9\\n\\\"q\\\"\"]},"
    "\"model.a.weight\":{\"dtype\":\"BF16\",\"shape\":[2,3],\"data_offsets\":[0,12]},"
    " \"b\" : {\"shape\":[],\"dtype\":\"F32\",\"data_offsets\":[12,16],\"extra\":{\"k\":[]}},\n"
    "\"c\":{\"dtype\":\"I8\",\"shape\":[4],\"data_offsets\":[16,20]}}";

static void test_header_valid() {
    const std::string img = file_image(kHeader, 20);
    std::vector<st::Tensor> ts;
    uint64_t off = 0;
    std::string err;
    CHECK(parse_exact(img, ts, &off, err), "valid header rejected: %s", err.c_str());
    CHECK(ts.size() == 3, "3 tensors expected, got %zu", ts.size());
    if (ts.size() != 3) return;
    CHECK(off == 8 + std::strlen(kHeader), "data offset %llu", (unsigned long long)off);
    CHECK(ts[0].name == "model.a.weight" && ts[0].dtype == SF_BF16, "entry 0");
    CHECK(ts[0].shape == std::vector<int64_t>({2, 3}) && ts[0].begin == 0 && ts[0].end == 12, "entry 0 shape");
    CHECK(ts[1].name == "b" && ts[1].dtype == SF_F32 && ts[1].shape.empty(), "entry 1");
    CHECK(ts[2].name == "c" && ts[2].dtype == SF_I8 && ts[2].end == 20, "entry 2");

    // Empty object, and an object holding only metadata.
    CHECK(parse_exact(file_image("{}", 0), ts, &off, err) && ts.empty(), "empty header");
    CHECK(parse_exact(file_image("{\"__metadata__\":{}}", 0), ts, &off, err) && ts.empty(), "metadata only");
}

static void test_header_truncations() {
    const std::string img = file_image(kHeader, 20);
    const size_t hend = 8 + std::strlen(kHeader);
    std::vector<st::Tensor> ts;
    uint64_t off;
    std::string err;
    for (size_t n = 0; n < img.size(); ++n) {
        const bool ok = parse_exact(img.substr(0, n), ts, &off, err);
        // The header itself cut short must fail; a short data section is
        // the loader's check (data range against file size), not the parser's.
        if (n < hend) CHECK(!ok, "truncation at %zu accepted", n);
    }
    // Header length field cut at every length inside the JSON text.
    for (size_t hl = 0; hl < std::strlen(kHeader); ++hl) {
        std::string cut = file_image(std::string(kHeader, hl), 0);
        CHECK(!parse_exact(cut, ts, &off, err), "header of %zu bytes accepted", hl);
    }
}

static void test_header_mutations() {
    const std::string base = file_image(kHeader, 20);
    const size_t hlen = std::strlen(kHeader);
    const char subs[] = {'"', '{', '}', '[', ']', ',', ':', '\\', '-', '0', '9', 'e', '.', ' ',
                         'u', 'n', '\0', '\x7f', '\xff', '\x80'};
    std::vector<st::Tensor> ts;
    uint64_t off;
    std::string err;
    size_t runs = 0;
    for (size_t pos = 8; pos < 8 + hlen; ++pos) {
        for (char c : subs) {
            std::string m = base;
            m[pos] = c;
            (void)parse_exact(m, ts, &off, err);
            ++runs;
        }
        std::string d = base;   // deletion, header length unchanged and adjusted
        d.erase(pos, 1);
        (void)parse_exact(d, ts, &off, err);
        uint64_t hl = hlen - 1;
        std::memcpy(&d[0], &hl, 8);
        (void)parse_exact(d, ts, &off, err);
        runs += 2;
    }
    for (int it = 0; it < 20000; ++it) {
        std::string m = base;
        const int nmut = 1 + (int)(next_u64() % 4);
        for (int k = 0; k < nmut; ++k) {
            const size_t pos = (size_t)(next_u64() % m.size());
            m[pos] = (char)(next_u64() & 0xff);
        }
        if (next_u64() % 8 == 0) m.resize((size_t)(next_u64() % m.size()));
        (void)parse_exact(m, ts, &off, err);
        ++runs;
    }
    std::printf("header mutations: %zu parses\n", runs);
}

static void test_header_limits() {
    std::vector<st::Tensor> ts;
    uint64_t off;
    std::string err;
    auto meta = [](int depth) {
        return "{\"__metadata__\":" + std::string(depth, '[') + std::string(depth, ']') + "}";
    };
    CHECK(parse_exact(file_image(meta(60), 0), ts, &off, err), "nesting 60 rejected: %s", err.c_str());
    CHECK(!parse_exact(file_image(meta(100000), 0), ts, &off, err), "nesting 100000 accepted");
    auto entry = [](const std::string& shape, const std::string& offs) {
        return "{\"t\":{\"dtype\":\"F32\",\"shape\":" + shape + ",\"data_offsets\":" + offs + "}}";
    };
    CHECK(parse_exact(file_image(entry("[1]", "[0,4611686018427387904]"), 0), ts, &off, err),
          "offset 2^62 rejected");
    CHECK(!parse_exact(file_image(entry("[1]", "[0,4611686018427387905]"), 0), ts, &off, err),
          "offset 2^62+1 accepted");
    CHECK(!parse_exact(file_image(entry("[1]", "[0,99999999999999999999999]"), 0), ts, &off, err),
          "offset past 64 bits accepted");
    CHECK(!parse_exact(file_image(entry("[1]", "[0,18446744073709551617]"), 0), ts, &off, err),
          "offset 2^64+1 accepted");
    CHECK(!parse_exact(file_image(entry("[1]", "[-1,4]"), 0), ts, &off, err), "negative offset accepted");
    CHECK(!parse_exact(file_image(entry("[1]", "[8,4]"), 0), ts, &off, err), "reversed offsets accepted");
    CHECK(!parse_exact(file_image(entry("[1]", "[0,4,8]"), 0), ts, &off, err), "3 offsets accepted");
    CHECK(!parse_exact(file_image(entry("[-2]", "[0,4]"), 0), ts, &off, err), "negative dim accepted");
    CHECK(!parse_exact(file_image(entry("[1.5]", "[0,4]"), 0), ts, &off, err), "fractional dim accepted");
    CHECK(!parse_exact(file_image("{\"t\":{\"dtype\":\"F32\",\"shape\":[1]}}", 0), ts, &off, err),
          "entry without offsets accepted");
    // Length field larger than the file, and the largest 64-bit value.
    std::string img = file_image("{}", 0);
    for (uint64_t hl : {(uint64_t)3, (uint64_t)1 << 40, ~(uint64_t)0}) {
        std::memcpy(&img[0], &hl, 8);
        CHECK(!parse_exact(img, ts, &off, err), "length %llu accepted", (unsigned long long)hl);
    }
    // Unknown dtype parses (code -1): the loader rejects it per tensor.
    CHECK(parse_exact(file_image("{\"t\":{\"dtype\":\"F8_E4M3\",\"shape\":[1],\"data_offsets\":[0,1]}}", 1),
                      ts, &off, err) && ts.size() == 1 && ts[0].dtype == -1,
          "unknown dtype");
}

static void test_inspect_file() {
    char path[] = "/tmp/sf_sanitize_XXXXXX";
    const int fd = mkstemp(path);
    CHECK(fd >= 0, "mkstemp");
    if (fd < 0) return;
    const std::string img = file_image(kHeader, 20);
    CHECK(write(fd, img.data(), img.size()) == (ssize_t)img.size(), "write");
    close(fd);
    int32_t count = -1;
    CHECK(sf_safetensors_inspect(path, nullptr, 0, &count) == SF_OK && count == 3, "inspect count");
    sf_st_entry e[8];
    CHECK(sf_safetensors_inspect(path, e, 2, &count) == SF_OK && count == 3, "inspect 2 entries");
    CHECK(std::strcmp(e[0].name, "model.a.weight") == 0 && e[0].ndim == 2 && e[0].shape[1] == 3,
          "inspect entry 0");
    const uint64_t off = 8 + std::strlen(kHeader);
    CHECK(e[1].data_begin == off + 12 && e[1].data_end == off + 16 && e[1].ndim == 0, "inspect entry 1");
    CHECK(sf_safetensors_inspect(path, e, 8, &count) == SF_OK && e[2].dtype == SF_I8, "inspect 8 entries");
    CHECK(sf_safetensors_inspect(path, nullptr, 2, &count) == SF_EINVAL, "null entries accepted");
    CHECK(sf_safetensors_inspect("/nonexistent/x.safetensors", e, 8, &count) == SF_EINVAL, "missing file");
    // A name longer than the entry's 256 bytes is cut, NUL-terminated.
    const std::string longname(1000, 'n');
    const std::string img2 = file_image("{\"" + longname + "\":{\"dtype\":\"F32\",\"shape\":[1],\"data_offsets\":[0,4]}}", 4);
    FILE* f = std::fopen(path, "wb");
    std::fwrite(img2.data(), 1, img2.size(), f);
    std::fclose(f);
    CHECK(sf_safetensors_inspect(path, e, 8, &count) == SF_OK && count == 1 && std::strlen(e[0].name) == 255,
          "long name");
    f = std::fopen(path, "wb");   // empty file
    std::fclose(f);
    CHECK(sf_safetensors_inspect(path, e, 8, &count) == SF_EINVAL, "empty file accepted");
    unlink(path);
}

static void test_conversions() {
    // fp16 codes against the closed form: subnormal m * 2^-24, normal
    // (1024 + m) * 2^(e - 25), e = 31 inf / NaN.
    for (uint32_t h = 0; h < 65536; ++h) {
        const uint32_t e = (h >> 10) & 31, m = h & 1023;
        const float sgn = (h & 0x8000) ? -1.f : 1.f;
        const float got = st::f16_to_f32((uint16_t)h);
        if (e == 31) {
            CHECK(m ? std::isnan(got) : (std::isinf(got) && std::signbit(got) == (sgn < 0)), "f16 %04x", h);
            continue;
        }
        const double want = sgn * (e == 0 ? std::ldexp((double)m, -24) : std::ldexp(1024.0 + m, (int)e - 25));
        CHECK((double)got == want && std::signbit(got) == (sgn < 0), "f16 %04x: %g vs %g", h, got, want);
    }
    // bf16 rounding against the oracle's independent restatement.
    const float vals[] = {0.f, -0.f, 1.f, 1.00390625f, 1.005859375f, 3.0e38f, -3.4e38f, 1e-40f,
                          INFINITY, -INFINITY, NAN, 65504.f, 2.5f, -7.75e-3f};
    for (float v : vals) {
        const uint16_t b = st::f32_to_bf16(v);
        const float r = sfo_bf16_round(v);
        uint32_t rb;
        std::memcpy(&rb, &r, 4);
        if (std::isnan(v)) CHECK(((b >> 7) & 0xff) == 0xff && (b & 0x7f), "bf16 NaN");
        else CHECK(b == (uint16_t)(rb >> 16), "bf16 of %g: %04x vs %04x", v, b, (unsigned)(rb >> 16));
    }
    // Unaligned sources.
    std::vector<char> raw(1 + 4 * 5);
    const float src[5] = {1.5f, -2.f, 3.25f, 0.f, 1e-3f};
    std::memcpy(raw.data() + 1, src, sizeof src);
    std::vector<float> out;
    st::to_f32(raw.data() + 1, SF_F32, 5, out);
    CHECK(std::memcmp(out.data(), src, sizeof src) == 0, "f32 unaligned");
    const uint16_t h16[3] = {0x3c00, 0xc000, 0x0001};
    std::memcpy(raw.data() + 1, h16, sizeof h16);
    st::to_f32(raw.data() + 1, SF_F16, 3, out);
    CHECK(out[0] == 1.f && out[1] == -2.f && out[2] == std::ldexp(1.f, -24), "f16 unaligned");
    const uint16_t b16[2] = {0x3f80, 0xbfc0};
    std::memcpy(raw.data() + 1, b16, sizeof b16);
    st::to_f32(raw.data() + 1, SF_BF16, 2, out);
    CHECK(out[0] == 1.f && out[1] == -1.5f, "bf16 unaligned");

    CHECK(st::remap_key("model.blocks.0.attn.qkv.weight") == "blocks.0.attn.qkv.weight", "remap model.");
    CHECK(st::remap_key("ema_model.x").empty() && st::remap_key("a.shadow_params.0").empty(), "remap ema");
    CHECK(st::remap_key("optimizer.state").empty() && st::remap_key("lr_scheduler.x").empty(), "remap opt");
    CHECK(st::same_shape({1, 67, 2048}, {67, 2048}) && !st::same_shape({2, 67}, {67}), "same_shape");
    CHECK(st::same_shape({1}, {1}) && st::same_shape({1, 1}, {1}) && !st::same_shape({}, {0}), "same_shape 1");
    CHECK(st::dtype_code("bfloat16") == SF_BF16 && st::dtype_code("bf16") == -1 && st::dtype_bytes(-1) == 0,
          "dtype codes");
}

static void test_oracle() {
    // Attention: fp32 online softmax against the fp64 two-pass form.
    const int shapes[][5] = {{1, 1, 1, 1, 1}, {2, 3, 5, 7, 8}, {1, 2, 3, 33, 64}, {2, 1, 9, 4, 16}};
    for (const auto& s : shapes) {
        const int B = s[0], H = s[1], Sq = s[2], Sk = s[3], D = s[4];
        std::vector<float> q((size_t)B * H * Sq * D), k((size_t)B * H * Sk * D), v(k.size()), o(q.size());
        std::vector<double> o64(q.size());
        sfo_randn(1, (int64_t)q.size(), 1.f, q.data());
        sfo_randn(2, (int64_t)k.size(), 1.f, k.data());
        sfo_randn(3, (int64_t)v.size(), 1.f, v.data());
        std::vector<int32_t> vl(B);
        for (int causal = 0; causal < 2; ++causal) {
            for (int mode = 0; mode < 4; ++mode) {
                for (int b = 0; b < B; ++b) vl[b] = mode == 0 ? 0 : mode == 1 ? Sk + 5 : mode == 2 ? -3 : (b + 1) % (Sk + 1);
                const int32_t* vlp = mode == 3 && causal ? nullptr : vl.data();
                sfo_attention_f32(q.data(), k.data(), v.data(), o.data(), B, H, Sq, Sk, D, 0.f, causal, vlp);
                sfo_attention_f64(q.data(), k.data(), v.data(), o64.data(), B, H, Sq, Sk, D, 0.0, causal, vlp);
                double err = 0;
                for (size_t i = 0; i < o.size(); ++i) err = std::fmax(err, std::fabs(o[i] - o64[i]));
                CHECK(err < 1e-5, "attention B%d H%d Sq%d Sk%d D%d causal %d mode %d: %g", B, H, Sq, Sk, D,
                      causal, mode, err);
                if (mode == 0 || mode == 2)
                    for (float x : o) CHECK(x == 0.f, "empty key set gives zeros");
            }
        }
    }
    // Norms, one-column and ragged rows.
    for (int64_t cols : {1, 37}) {
        const int64_t rows = 3, n = rows * cols;
        std::vector<float> x(n), g(cols), r(n), out(n), in(n);
        sfo_randn(4, n, 1.f, x.data());
        sfo_randn(5, cols, 1.f, g.data());
        sfo_randn(6, n, 1.f, in.data());
        sfo_rms_norm(x.data(), g.data(), out.data(), rows, cols, 1e-6f);
        for (int64_t i = 0; i < n; ++i) CHECK(std::isfinite(out[i]), "rms_norm finite");
        r = x;
        sfo_fused_add_rms_norm(in.data(), r.data(), g.data(), out.data(), rows, cols, 1e-6f);
        for (int64_t i = 0; i < n; ++i) CHECK(r[i] == x[i] + in[i], "residual add");
    }
    // Linear with and without bias, each activation, K not a multiple of 8.
    {
        const int64_t M = 3, N = 5, K = 13;
        std::vector<float> x(M * K), w(N * K), b(N), y(M * N);
        sfo_randn(7, M * K, 1.f, x.data());
        sfo_randn(8, N * K, 1.f, w.data());
        sfo_randn(9, N, 1.f, b.data());
        for (int act = 0; act < 3; ++act) {
            sfo_linear(x.data(), w.data(), act ? b.data() : nullptr, y.data(), M, N, K, act);
            double ref = 0;
            for (int64_t kk = 0; kk < K; ++kk) ref += (double)x[kk] * w[kk];
            if (act) ref += b[0];
            if (act == 1) ref = 0.5 * ref * (1 + std::tanh(std::sqrt(2 / M_PI) * (ref + 0.044715 * ref * ref * ref)));
            if (act == 2) ref = ref / (1 + std::exp(-ref));
            CHECK(std::fabs(y[0] - ref) < 1e-4, "linear act %d: %g vs %g", act, y[0], ref);
        }
    }
    // Layout maps: seq_to_head / head_to_seq round trip, split_qkv / split_kv slices.
    {
        const int B = 2, S = 3, H = 2, D = 5;
        const int64_t n = (int64_t)B * S * H * D;
        std::vector<float> a(n), h(n), back(n), qkv(3 * n), Q(n), K(n), V(n), K2(n), V2(n), kv(2 * n);
        for (int64_t i = 0; i < n; ++i) a[i] = (float)i;
        for (int64_t i = 0; i < 3 * n; ++i) qkv[i] = (float)i;
        for (int64_t i = 0; i < 2 * n; ++i) kv[i] = (float)i;
        sfo_seq_to_head(a.data(), h.data(), B, S, H, D);
        sfo_head_to_seq(h.data(), back.data(), B, H, S, D);
        CHECK(a == back, "seq_to_head round trip");
        sfo_split_qkv(qkv.data(), Q.data(), K.data(), V.data(), B, S, H, D);
        sfo_split_kv(kv.data(), K2.data(), V2.data(), B, S, H, D);
        // [b=1, h=1, s=2, d=4]: source row (b*S + s) of width 3HD / 2HD.
        const int64_t idx = ((1 * H + 1) * S + 2) * D + 4, row = 1 * S + 2;
        CHECK(Q[idx] == row * 3 * H * D + 1 * D + 4 && V[idx] == row * 3 * H * D + (2 * H + 1) * D + 4, "split_qkv");
        CHECK(K2[idx] == row * 2 * H * D + 1 * D + 4 && V2[idx] == row * 2 * H * D + (H + 1) * D + 4, "split_kv");
    }
    // int8: all-zero row (scale 1), round trip within half a step.
    {
        const int64_t N = 3, K = 11;
        std::vector<float> w(N * K), deq(N * K), sc(N);
        std::vector<int8_t> qv(N * K);
        sfo_randn(10, N * K, 1.f, w.data());
        for (int64_t c = 0; c < K; ++c) w[K + c] = 0.f;
        sfo_quantize_int8_rows(w.data(), N, K, qv.data(), sc.data());
        CHECK(sc[1] == 1.f, "zero row scale");
        sfo_dequant_int8(qv.data(), sc.data(), deq.data(), N, K, 1);
        for (int64_t i = 0; i < N * K; ++i)
            CHECK(std::fabs(deq[i] - w[i]) <= 0.5f * sc[i / K] * 1.0001f, "int8 round trip %lld", (long long)i);
        sfo_dequant_int8(qv.data(), sc.data(), deq.data(), N, K, 0);
        CHECK(deq[2] == (float)qv[2] * sc[0], "per-tensor dequant");
    }
    // Schedule, sincos table (odd width leaves the last column), timestep index.
    {
        std::vector<float> t(2);
        sfo_linspace(1, 1.f, 0.f, t.data());
        CHECK(t[0] == 1.f && t[1] == 0.f, "linspace 1 step");
        std::vector<float> tab(4 * 7, -9.f);
        sfo_sincos_table(4, 7, tab.data());
        CHECK(tab[0] == 1.f && tab[3] == 0.f && tab[6] == -9.f, "sincos odd width");
        CHECK(sfo_timestep_index(-1.f, 1000) == 0 && sfo_timestep_index(2.f, 1000) == 999, "timestep clamp");
        CHECK(sfo_timestep_index(0.5f, 1000) == 500 && sfo_timestep_index(1.f, 1) == 0, "timestep index");
    }
}

int main() {
    test_header_valid();
    test_header_truncations();
    test_header_mutations();
    test_header_limits();
    test_inspect_file();
    test_conversions();
    test_oracle();
    if (g_fail) {
        std::printf("%d check(s) failed\n", g_fail);
        return 1;
    }
    std::printf("sanitize_host: all checks passed\n");
    return 0;
}
