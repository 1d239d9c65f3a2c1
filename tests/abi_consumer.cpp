// A compiled C++ consumer of the C ABI (include/nsosx.h) through the host
// mirror (reimagined_amd/host/nsosx.hpp), the way a C++ caller of the
// reference's BitLinear would bind it.  Built by the tests with
// g++ -Wall -Werror (tests/test_abi_consumer.py) and by the package build.
//
//   abi_consumer cpu <edge_pack_file>   host entry points only: packer, unpacker,
//                                       SHA-256, edge pack parse, error mapping
//   abi_consumer gpu <out_file>         BitLinear forward (packed and float
//                                       paths) on the device; writes inputs and
//                                       outputs as float32 for the test's oracle
//   abi_consumer bench <K> <N>          back-to-back quantize + GEMV calls on one
//                                       resident weight set (M = 1), host wall
//                                       time per call, the reference's own method
//                                       (benchmarks/bench_decode_gemv.cpp:76-90)
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <fstream>
#include <iterator>
#include <string>
#include <vector>

#include "nsosx.hpp"

namespace {

std::vector<float> lcg_ternary(size_t n, uint32_t seed) {
    std::vector<float> w(n);
    uint32_t r = seed;
    for (auto& v : w) {
        r = r * 1664525u + 1013904223u;
        v = static_cast<float>(static_cast<int>((r >> 16) % 3) - 1);
    }
    return w;
}

std::vector<float> waves(size_t n, float a, float b) {
    std::vector<float> x(n);
    for (size_t i = 0; i < n; ++i)
        x[i] = std::sin(static_cast<float>(i) * a) + 0.25f * std::cos(static_cast<float>(i) * b);
    return x;
}

int run_cpu(const char* pack_path) {
    std::printf("{\"version\": \"%s\"", nsosx_version());
    // BitLinear::pack_weights on a small ternary-valued matrix
    const int N = 24, K = 48;
    std::vector<float> w = lcg_ternary((size_t)N * K, 20260919u);
    for (size_t i = 0; i < w.size(); ++i) w[i] *= 0.5f + 0.01f * static_cast<float>(i % 7);
    std::vector<uint32_t> packed((size_t)N * K / 16);
    float ws = 0.0f;
    nsosx::check(nsosx_pack_ternary(w.data(), N, K, packed.data(), &ws), "pack_ternary");
    uint32_t bits;
    std::memcpy(&bits, &ws, 4);
    std::printf(", \"weight_scale_bits\": %u, \"packed\": [", bits);
    for (size_t i = 0; i < packed.size(); ++i) std::printf("%s%u", i ? ", " : "", packed[i]);
    std::vector<int8_t> codes((size_t)N * K);
    nsosx::check(nsosx_unpack_ternary(packed.data(), (int64_t)codes.size(), codes.data()),
                 "unpack_ternary");
    long code_sum = 0;
    for (int8_t c : codes) code_sum += c;
    std::printf("], \"code_sum\": %ld", code_sum);
    // SHA-256 of "abc" and of the pack file
    char hex[65];
    nsosx::check(nsosx_sha256_hex(reinterpret_cast<const uint8_t*>("abc"), 3, hex), "sha256");
    std::printf(", \"sha256_abc\": \"%s\"", hex);
    std::ifstream f(pack_path, std::ios::binary);
    std::vector<uint8_t> blob((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    nsosx::check(nsosx_sha256_hex(blob.data(), blob.size(), hex), "sha256");
    std::printf(", \"sha256_pack\": \"%s\"", hex);
    int count = 0;
    uint32_t version = 0;
    (void)nsosx_edge_pack_parse(blob.data(), blob.size(), nullptr, 0, &count, &version);
    std::vector<nsosx_edge_layer> layers(count);
    nsosx::check(nsosx_edge_pack_parse(blob.data(), blob.size(), layers.data(), count, &count,
                                       &version),
                 "edge_pack_parse");
    std::printf(", \"edge_version\": %u, \"edge_layers\": [", version);
    for (int i = 0; i < count; ++i) {
        const auto& L = layers[i];
        std::printf("%s{\"in\": %d, \"out\": %d, \"use_bias\": %d, \"sensitive\": %d, "
                    "\"packed_words\": %llu, \"packed_offset\": %llu}",
                    i ? ", " : "", L.in_features, L.out_features, L.use_bias, L.sensitive,
                    (unsigned long long)L.packed_words, (unsigned long long)L.packed_offset);
    }
    // the facade maps statuses to the reference's exception types
    std::string mapped = "none";
    try {
        nsosx::check(nsosx_pack_ternary(w.data(), N, 10, packed.data(), &ws), "pack_ternary");
    } catch (const std::invalid_argument&) {
        mapped = "invalid_argument";
    }
    std::printf("], \"bad_shape_throws\": \"%s\"}\n", mapped.c_str());
    return 0;
}

int run_gpu(const char* out_path) {
    const int M = 33, K = 256, N = 96;
    std::vector<float> x = waves((size_t)M * K, 0.013f, 0.037f);
    std::vector<float> w = lcg_ternary((size_t)N * K, 7u);
    for (size_t i = 0; i < w.size(); ++i) w[i] *= 0.02f + 0.001f * static_cast<float>(i % 13);
    std::vector<float> mag(N), bias(N);
    for (int n = 0; n < N; ++n) {
        mag[n] = 0.75f + 0.005f * static_cast<float>(n);
        bias[n] = 0.1f * std::sin(static_cast<float>(n));
    }
    nsosx::DeviceBuffer xd, yd(sizeof(float) * M * N);
    xd.upload(x);
    nsosx::BitLinear bl(K, N, true);
    bl.set_weights(w);
    bl.set_magnitude(mag);
    bl.set_bias(bias);
    bl.forward(xd.data(), NSOSX_F32, M, yd.data(), NSOSX_F32);
    std::vector<float> y_packed = yd.download<float>((size_t)M * N);
    bl.set_quantization_sensitive(true);
    bl.forward(xd.data(), NSOSX_F32, M, yd.data(), NSOSX_F32);
    std::vector<float> y_float = yd.download<float>((size_t)M * N);
    // import_packed_state rejects a reserved code
    nsosx::PackedState st = bl.export_packed_state();
    st.packed_weights[5] |= 0x3u << 6;
    std::string rejected = "no";
    nsosx::BitLinear other(K, N, true);
    try {
        other.import_packed_state(st);
    } catch (const std::invalid_argument&) {
        rejected = "invalid_argument";
    }
    std::ofstream f(out_path, std::ios::binary);
    for (const auto* v : {&x, &w, &mag, &bias, &y_packed, &y_float})
        f.write(reinterpret_cast<const char*>(v->data()), (std::streamsize)(v->size() * 4));
    std::printf("{\"M\": %d, \"K\": %d, \"N\": %d, \"reserved_code_import\": \"%s\"}\n", M, K, N,
                rejected.c_str());
    return 0;
}

int run_bench(int K, int N) {
    nsosx::BitLinear bl(K, N, false);
    bl.set_exact_linear_mode(true);  // the reference benchmark quantizes raw x (no RMSNorm)
    bl.set_weights(lcg_ternary((size_t)N * K, 20260919u));
    nsosx::DeviceBuffer xd, yd(sizeof(float) * N);
    xd.upload(waves(K, 0.013f, 0.037f));
    constexpr int warmup = 20, iterations = 100, repeats = 7;
    for (int i = 0; i < warmup; ++i) bl.forward(xd.data(), NSOSX_F32, 1, yd.data(), NSOSX_F32);
    nsosx::check_hip(hipDeviceSynchronize(), "sync");
    std::vector<double> wall;
    for (int r = 0; r < repeats; ++r) {
        const auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < iterations; ++i)
            bl.forward(xd.data(), NSOSX_F32, 1, yd.data(), NSOSX_F32);
        nsosx::check_hip(hipDeviceSynchronize(), "sync");
        wall.push_back(std::chrono::duration<double, std::micro>(
                           std::chrono::steady_clock::now() - t0).count() / iterations);
    }
    std::sort(wall.begin(), wall.end());
    std::printf("{\"K\": %d, \"N\": %d, \"median_wall_us\": %.3f, \"min_wall_us\": %.3f}\n", K, N,
                wall[wall.size() / 2], wall.front());
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    try {
        const std::string mode = argc > 1 ? argv[1] : "";
        if (mode == "cpu" && argc == 3) return run_cpu(argv[2]);
        if (mode == "gpu" && argc == 3) return run_gpu(argv[2]);
        if (mode == "bench" && argc == 4) return run_bench(std::stoi(argv[2]), std::stoi(argv[3]));
        std::fprintf(stderr, "usage: abi_consumer cpu <pack> | gpu <out> | bench <K> <N>\n");
        return 2;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "abi_consumer: %s\n", e.what());
        return 1;
    }
}
