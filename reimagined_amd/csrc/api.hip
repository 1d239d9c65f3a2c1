// Host-side part of the nsosx C ABI: error text, version, and the weight
// packer/unpacker that prepares BitLinear weights before upload.
#include "common.hpp"

#include <cmath>
#include <cstring>
#include <string>

namespace nsosx {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

}  // namespace nsosx

using namespace nsosx;

extern "C" const char* nsosx_last_error(void) { return g_last_error.c_str(); }

extern "C" const char* nsosx_version(void) { return "nsosx 0.1 gfx950"; }

// BitLinear::pack_weights (OXN/nsos/src/bitlinear.cpp:152-193): absmean in
// double (tensor_abs_mean, src/tensor.cpp:2096-2107) plus 1e-8f, then the
// ternary rule of quantize_weights (src/bitlinear.cpp:1359-1379) with the
// 1e-8f added a second time, packed 16 codes per word, code j at bits 2j
// (BitNetAdapter::pack_weights_microsoft_style, src/bitnet_adapter.cpp:570-588).
extern "C" int nsosx_pack_ternary(const float* w, int N, int K, uint32_t* packed,
                                  float* weight_scale) {
    if (!w || !packed || !weight_scale) return fail(NSOSX_ERR_INVALID, "pack_ternary: null pointer");
    if (N <= 0 || K <= 0 || K % 16 != 0)
        return fail(NSOSX_ERR_INVALID, "pack_ternary: need N > 0 and K a positive multiple of 16");
    const int64_t n = (int64_t)N * K;
    double total = 0.0;
    for (int64_t i = 0; i < n; ++i) total += std::fabs(static_cast<double>(w[i]));
    const float absmean = static_cast<float>(total / static_cast<double>(n));
    const float ws = absmean + 1e-8f;
    const float denom = ws + 1e-8f;
    std::memset(packed, 0, sizeof(uint32_t) * (size_t)(n / 16));
    for (int64_t i = 0; i < n; ++i) {
        const float v = w[i] / denom;
        const uint32_t two = v > 0.5f ? 2u : (v < -0.5f ? 0u : 1u);
        packed[i >> 4] |= two << ((i & 15) * 2);
    }
    *weight_scale = ws;
    return NSOSX_OK;
}

// BitNetAdapter::unpack_weights_microsoft_style_to_i8 with the decode table
// {-1, 0, +1, 0} (src/bitnet_adapter.cpp:31,590-606).
extern "C" int nsosx_unpack_ternary(const uint32_t* packed, int64_t n, int8_t* codes) {
    if (!packed || !codes || n < 0) return fail(NSOSX_ERR_INVALID, "unpack_ternary: bad argument");
    static const int8_t lut[4] = {-1, 0, 1, 0};
    for (int64_t i = 0; i < n; ++i) codes[i] = lut[(packed[i >> 4] >> ((i & 15) * 2)) & 3u];
    return NSOSX_OK;
}
