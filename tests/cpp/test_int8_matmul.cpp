// C++ host-layer tests, mirroring crates/omni-kernel/src/int8_matmul.rs:605-786
// (the reference's own tests) through include/omni_kernel.hpp. The expected
// values come from the CPU oracle (test infrastructure, oracle/). Needs a
// gfx950 GPU; prints one line per test and exits non-zero on any failure.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../../include/omni_kernel.hpp"
#include "../../oracle/oracle_int8.h"

using omni_kernel::DeviceTensor;
using omni_kernel::DType;

static int g_failures = 0;
#define EXPECT(cond, ...)                                   \
    do {                                                    \
        if (!(cond)) {                                      \
            std::printf("  FAIL %s:%d: ", __FILE__, __LINE__); \
            std::printf(__VA_ARGS__);                       \
            std::printf("\n");                              \
            ++g_failures;                                   \
        }                                                   \
    } while (0)

template <typename T>
static DeviceTensor upload(const std::vector<T>& host, std::vector<int64_t> shape, DType dt) {
    void* p = nullptr;
    if (hipMalloc(&p, host.size() * sizeof(T) + 16) != hipSuccess) std::abort();
    if (hipMemcpy(p, host.data(), host.size() * sizeof(T), hipMemcpyHostToDevice) != hipSuccess) std::abort();
    return DeviceTensor{p, std::move(shape), dt};
}

template <typename T>
static std::vector<T> download(const DeviceTensor& t) {
    std::vector<T> host((size_t)t.numel());
    if (hipDeviceSynchronize() != hipSuccess) std::abort();
    if (hipMemcpy(host.data(), t.data, host.size() * sizeof(T), hipMemcpyDeviceToHost) != hipSuccess) std::abort();
    return host;
}

static std::vector<int32_t> pack(const std::vector<int8_t>& codes) {
    std::vector<int32_t> words(codes.size() / 4);
    oracle_pack_i8(codes.data(), (int64_t)codes.size(), words.data());
    return words;
}

// Runs try_int8_gemm on host inputs; returns the f32 output.
static std::vector<float> run_gemm(const std::vector<float>& x, int64_t rows, int64_t width,
                                   const std::vector<int8_t>& w, const std::vector<float>& scale,
                                   const std::vector<int32_t>& zero) {
    omni_kernel::HipAllocator alloc;
    const int64_t columns = (int64_t)scale.size();
    auto dx = upload(x, {rows, width}, DType::F32);
    auto dw = upload(pack(w), {columns * width / 4}, DType::I32);
    auto ds = upload(scale, {columns}, DType::F32);
    auto dz = upload(zero, {columns}, DType::I32);
    auto out = omni_kernel::int8_matmul::try_int8_gemm(dx, dw, ds, dz, alloc);
    EXPECT(out.has_value(), "try_int8_gemm returned None");
    std::vector<float> host = out ? download<float>(*out) : std::vector<float>();
    if (out) alloc.release(out->data, nullptr);
    for (auto* t : {&dx, &dw, &ds, &dz}) (void)hipFree(t->data);
    return host;
}

// int8_matmul.rs:700-732 (host) and :749-786 (device): hand value -411/127
// and the got+1 negative control.
static void hand_value_matches_f16_dequantized_weights() {
    std::puts("hand_value_matches_f16_dequantized_weights");
    const std::vector<float> x{1.0f, -2.0f, 0.5f, 4.0f};
    const std::vector<int8_t> w{1, -2, 3, -4};
    const std::vector<float> scale{0.25f};
    const std::vector<int32_t> zero{1};
    float expected = 0.0f;
    oracle_dequant_reference(x.data(), 1, 4, w.data(), scale.data(), zero.data(), 1, &expected);
    EXPECT(std::fabs(expected - (-411.0f / 127.0f)) < 1e-5f, "reference %f", expected);
    const auto got = run_gemm(x, 1, 4, w, scale, zero);
    EXPECT(got.size() == 1 && std::fabs(got[0] - expected) < 1e-3f, "got %f want %f", got.empty() ? 0 : got[0], expected);
    EXPECT(!got.empty() && std::fabs(got[0] + 1.0f - expected) >= 1e-3f, "negative control passed");
}

// int8_matmul.rs:734-747: the 64x64x64 tile fixture.
static void tile64_fixture() {
    std::puts("tile64_fixture");
    std::vector<float> x(64 * 64, 0.0f);
    x[0] = 1.0f; x[1] = -2.0f; x[2] = 0.5f; x[3] = 4.0f;
    std::vector<int8_t> w(64 * 64, 0);
    w[0] = 1; w[1] = -2; w[2] = 3; w[3] = -4;
    std::vector<float> scale(64, 0.25f);
    std::vector<int32_t> zero(64, 0);
    zero[0] = 1;
    std::vector<float> expected(64 * 64);
    oracle_dequant_reference(x.data(), 64, 64, w.data(), scale.data(), zero.data(), 64, expected.data());
    EXPECT(std::fabs(expected[0] - (-411.0f / 127.0f)) < 1e-5f, "reference %f", expected[0]);
    const auto got = run_gemm(x, 64, 64, w, scale, zero);
    float worst = 0.0f;
    for (size_t i = 0; i < got.size(); ++i) worst = std::fmax(worst, std::fabs(got[i] - expected[i]));
    EXPECT(got.size() == expected.size() && worst < 1e-3f, "max |got - want| = %g", worst);
    EXPECT(!got.empty() && std::fabs(got[0] + 1.0f - expected[0]) >= 1e-3f, "negative control passed");
}

// prototypes/int8-gemm/src/main.rs:69-89: check shapes against the integer
// reference (int8_host.rs:19-53), bit-exact.
static void prototype_check_shapes() {
    std::puts("prototype_check_shapes");
    const int64_t shapes[2][3] = {{5, 12, 6}, {17, 36, 14}};
    for (const auto& sh : shapes) {
        const int64_t rows = sh[0], width = sh[1], columns = sh[2];
        std::vector<float> x(rows * width);
        for (int64_t i = 0; i < rows * width; ++i) x[i] = (float)((i * 17) % 41) - 20.0f;
        std::vector<int8_t> w(columns * width);
        for (int64_t i = 0; i < columns * width; ++i) w[i] = (int8_t)(((i * 13) % 31) - 15);
        std::vector<float> scale(columns);
        std::vector<int32_t> zero(columns);
        for (int64_t i = 0; i < columns; ++i) {
            scale[i] = 0.05f + (float)i * 0.01f;
            zero[i] = (int32_t)(i % 5) - 2;
        }
        std::vector<float> want(rows * columns);
        oracle_int8_gemm(x.data(), rows, width, w.data(), scale.data(), zero.data(), columns, want.data());
        const auto got = run_gemm(x, rows, width, w, scale, zero);
        EXPECT(got.size() == want.size() && std::memcmp(got.data(), want.data(), got.size() * 4) == 0,
               "%lldx%lldx%lld not bit-exact", (long long)rows, (long long)width, (long long)columns);
    }
}

// int8_matmul.rs:517-521: shape disagreements return None.
static void shape_mismatch_returns_none() {
    std::puts("shape_mismatch_returns_none");
    omni_kernel::HipAllocator alloc;
    auto dx = upload(std::vector<float>(2 * 8, 0.0f), {2, 8}, DType::F32);
    auto dw = upload(std::vector<int32_t>(3, 0), {3}, DType::I32);  // want 2 * 8 / 4 = 4
    auto ds = upload(std::vector<float>(2, 1.0f), {2}, DType::F32);
    auto dz = upload(std::vector<int32_t>(2, 0), {2}, DType::I32);
    EXPECT(!omni_kernel::int8_matmul::try_int8_gemm(dx, dw, ds, dz, alloc).has_value(), "packed length");
    auto dz3 = upload(std::vector<int32_t>(3, 0), {3}, DType::I32);
    auto dw4 = upload(std::vector<int32_t>(4, 0), {4}, DType::I32);
    EXPECT(!omni_kernel::int8_matmul::try_int8_gemm(dx, dw4, ds, dz3, alloc).has_value(), "zero length");
    auto dx6 = upload(std::vector<float>(2 * 6, 0.0f), {2, 6}, DType::F32);
    EXPECT(!omni_kernel::int8_matmul::try_int8_gemm(dx6, dw, ds, dz, alloc).has_value(), "width %% 4");
    for (auto* t : {&dx, &dw, &ds, &dz, &dz3, &dw4, &dx6}) (void)hipFree(t->data);
}

// W8A16 linear against the f64 ground truth (1e-2, fp16 output).
static void w8a16_linear_matches_ground_truth() {
    std::puts("w8a16_linear_matches_ground_truth");
    omni_kernel::HipAllocator alloc;
    // The last two shapes split K through the workspace (the GEMM, and the
    // 5..16-row kernel when its 16-column units need more than one round).
    const int64_t cases[][3] = {{1, 512, 96}, {4, 512, 96}, {37, 512, 96}, {200, 8192, 160}, {16, 2048, 4200}};
    for (const auto& cs : cases) {
        const int64_t rows = cs[0], width = cs[1], columns = cs[2];
        std::vector<uint16_t> x(rows * width), scale(columns), bias(columns);
        std::vector<int8_t> w(columns * width);
        uint64_t st = 0x9e3779b97f4a7c15ull;
        auto rnd = [&]() { st ^= st << 13; st ^= st >> 7; st ^= st << 17; return st; };
        for (auto& v : x) v = oracle_f32_to_f16(((float)(rnd() % 2001) - 1000.0f) / 500.0f);
        for (auto& v : w) v = (int8_t)((int)(rnd() % 255) - 127);
        for (auto& v : scale) v = oracle_f32_to_f16(0.002f + (float)(rnd() % 1000) * 1.8e-5f);
        for (auto& v : bias) v = oracle_f32_to_f16(((float)(rnd() % 201) - 100.0f) / 50.0f);
        std::vector<double> ref(rows * columns);
        oracle_w8a16_f64(x.data(), rows, width, w.data(), scale.data(), bias.data(), columns, ref.data());
        auto dx = upload(x, {rows, width}, DType::F16);
        auto dw = upload(w, {columns, width}, DType::I8);
        auto ds = upload(scale, {columns}, DType::F16);
        auto db = upload(bias, {columns}, DType::F16);
        auto out = omni_kernel::w8a16_linear(dx, dw, ds, &db, alloc);
        const auto got = download<uint16_t>(out);
        double rms = 0.0;
        for (double r : ref) rms += r * r;
        rms = std::sqrt(rms / (double)ref.size());
        double worst = 0.0;
        for (size_t i = 0; i < got.size(); ++i) {
            const double g = oracle_f16_to_f32(got[i]);
            worst = std::fmax(worst, std::fabs(g - ref[i]) / std::fmax(std::fabs(ref[i]), 0.1 * rms));
        }
        EXPECT(worst <= 1e-2, "rows %lld: relative error %g", (long long)rows, worst);
        alloc.release(out.data, nullptr);
        for (auto* t : {&dx, &dw, &ds, &db}) (void)hipFree(t->data);
    }
}

int main() {
    if (!omni_kernel::device_supported()) {
        std::puts("no gfx950 device");
        return 2;
    }
    hand_value_matches_f16_dequantized_weights();
    tile64_fixture();
    prototype_check_shapes();
    shape_mismatch_returns_none();
    w8a16_linear_matches_ground_truth();
    std::printf("%s (%d failures)\n", g_failures ? "FAILED" : "OK", g_failures);
    return g_failures ? 1 : 0;
}
