// BitLinear on gfx950: the operator-level entry points (quantize + ternary GEMM
// dispatch by shape, the one-call forward) and the reserved-code import check.
// The kernels live in quant.hip (RMS_PERI + int8 codes), gemv.hip (the VALU
// GEMV), skinny.hip (the MFMA decode GEMV) and gemm.hip (the MFMA GEMMs).
//
// Reference semantics (OXN/nsos/ of vitorGgC569/reimagined):
//   quantization  src/bitlinear.cpp:240-291, src/bitlinear_quantize_avx2.cpp:65-103
//   RMS_PERI norm src/bitlinear.cpp:460-466, src/tensor.cpp:3455-3492
//   GEMM + affine src/bitnet_adapter_avx2.cpp:52-158
//   packed format src/bitnet_adapter.cpp:570-606
#include "bitlinear.hpp"

namespace nsosx {

// ===========================================================================
// Reserved-code scan (import check).
// ===========================================================================
__global__ void find_reserved_kernel(const uint32_t* __restrict__ packed, int64_t n_codes,
                                     unsigned long long* __restrict__ first_bad) {
    const int64_t words = (n_codes + 15) / 16;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < words;
         i += (int64_t)gridDim.x * blockDim.x) {
        const uint32_t p = packed[i];
        // a code is 3 when both of its bits are set
        uint32_t both = p & (p >> 1) & 0x55555555u;
        const int64_t valid = n_codes - i * 16;
        if (valid < 16) both &= (1u << (2 * valid)) - 1u;
        if (both) {
            const int j = __builtin_ctz(both) >> 1;
            atomicMin(first_bad, static_cast<unsigned long long>(i * 16 + j));
        }
    }
}

__global__ void finish_reserved_kernel(unsigned long long* v) {
    if (*v == ~0ull) *reinterpret_cast<long long*>(v) = -1;
}

__global__ void fill_u64_kernel(unsigned long long* p, unsigned long long v) { *p = v; }

}  // namespace nsosx

using namespace nsosx;

static int check_gemm_args(const int8_t* q, const float* as, const uint32_t* packed, float ws,
                           int M, int K, int N, const void* y, int y_dtype, const int32_t* acc) {
    if (!q || !as || !packed) return fail(NSOSX_ERR_INVALID, "ternary_gemm: null pointer");
    if (!y && !acc) return fail(NSOSX_ERR_INVALID, "ternary_gemm: no output");
    if (M <= 0 || K <= 0 || N <= 0) return fail(NSOSX_ERR_INVALID, "ternary_gemm: empty shape");
    if (K % 16 != 0) return fail(NSOSX_ERR_INVALID, "ternary_gemm: K must be a multiple of 16");
    if (!(ws > 0.0f) || !std::isfinite(ws))
        return fail(NSOSX_ERR_INVALID, "ternary_gemm: weight_scale must be finite and > 0");
    if (!valid_dtype(y_dtype)) return fail(NSOSX_ERR_INVALID, "ternary_gemm: bad dtype");
    if (K > 2147483647 / 254)  // |acc| <= 127 * K must fit int32 (bitnet_gpu_dispatch.cpp:97-101)
        return fail(NSOSX_ERR_OVERFLOW, "ternary_gemm: K too large for int32 accumulation");
    if ((int64_t)M * N > ((int64_t)1 << 40) || (int64_t)M * K > ((int64_t)1 << 40))
        return fail(NSOSX_ERR_OVERFLOW, "ternary_gemm: size too large");
    if (reinterpret_cast<uintptr_t>(q) % 16 || reinterpret_cast<uintptr_t>(packed) % 16)
        return fail(NSOSX_ERR_INVALID, "ternary_gemm: q and packed must be 16-byte aligned");
    return NSOSX_OK;
}

// M = 1: the VALU GEMV; 2 <= M <= 32 where the skinny MFMA path takes the
// shape; other M <= 8: the GEMV; else the MFMA GEMM.
static int ternary_gemm_auto_path(int M, int K, int N) {
    if (skinny_ok(M, K, N)) return 2;
    return M <= 8 ? 0 : 1;
}

extern "C" int nsosx_ternary_gemm_path(const int8_t* q, const float* act_scale,
                                       const uint32_t* packed, float weight_scale, int M, int K,
                                       int N, const float* magnitude, const float* bias, void* y,
                                       int y_dtype, int32_t* acc_out, int path, void* stream) {
    int rc = check_gemm_args(q, act_scale, packed, weight_scale, M, K, N, y, y_dtype, acc_out);
    if (rc) return rc;
    if (path == 0 && M > 8) return fail(NSOSX_ERR_INVALID, "ternary_gemm: GEMV path needs M <= 8");
    if (path < 0 || path > 2) return fail(NSOSX_ERR_INVALID, "ternary_gemm: bad path");
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (path == 2) {
        if (!skinny_ok(M, K, N))
            return fail(NSOSX_ERR_INVALID,
                        "ternary_gemm: skinny path needs 2 <= M <= 32, K in {1024, 2048, 4096}, "
                        "ceil(M / 16) * K <= 4096, M * N < 2^29");
        GemvProblem pb{packed, magnitude, bias, weight_scale, N, K};
        launch_skinny(pb, q, act_scale, M, y, y_dtype, acc_out, false, st);
    } else if (path == 0) {
        GemvProblem pb{packed, magnitude, bias, weight_scale, N, K};
        launch_gemv(pb, q, act_scale, M, y, y_dtype, acc_out, st);
    } else {
        GemmProblem pb{packed, magnitude, bias, weight_scale, N, K};
        launch_gemm(pb, q, act_scale, M, y, y_dtype, acc_out, st);
    }
    return check_launch("ternary_gemm");
}

extern "C" int nsosx_ternary_gemm(const int8_t* q, const float* act_scale, const uint32_t* packed,
                                  float weight_scale, int M, int K, int N, const float* magnitude,
                                  const float* bias, void* y, int y_dtype, int32_t* acc_out,
                                  void* stream) {
    return nsosx_ternary_gemm_path(q, act_scale, packed, weight_scale, M, K, N, magnitude, bias, y,
                                   y_dtype, acc_out, ternary_gemm_auto_path(M, K, N), stream);
}

extern "C" int nsosx_bitlinear_forward(const void* x, int x_dtype, const uint32_t* packed,
                                       float weight_scale, int M, int K, int N,
                                       int precision_bits, int rms_input, const float* magnitude,
                                       const float* bias, void* y, int y_dtype,
                                       int8_t* q_workspace, float* scale_workspace,
                                       float* rms_workspace, void* stream) {
    if (!y) return fail(NSOSX_ERR_INVALID, "bitlinear_forward: null output");
    int rc = check_gemm_args(q_workspace, scale_workspace, packed, weight_scale, M, K, N, y,
                             y_dtype, nullptr);
    if (rc) return rc;
    rc = nsosx_quantize_act_i8(x, x_dtype, M, K, precision_bits, rms_input, q_workspace,
                               scale_workspace, rms_workspace, stream);
    if (rc) return rc;
    return nsosx_ternary_gemm(q_workspace, scale_workspace, packed, weight_scale, M, K, N,
                              magnitude, bias, y, y_dtype, nullptr, stream);
}

extern "C" int nsosx_ternary_gemm_mfma(const int8_t* q, const float* act_scale,
                                       const uint32_t* packed_mfma, float weight_scale, int M,
                                       int K, int N, const float* magnitude, const float* bias,
                                       void* y, int y_dtype, int32_t* acc_out, void* stream) {
    int rc = check_gemm_args(q, act_scale, packed_mfma, weight_scale, M, K, N, y, y_dtype, acc_out);
    if (rc) return rc;
    if (K % kG3BK != 0)
        return fail(NSOSX_ERR_INVALID, "ternary_gemm_mfma: K must be a multiple of 128");
    if (K > kMfmaLayoutMaxK)
        return fail(NSOSX_ERR_OVERFLOW, "ternary_gemm_mfma: K too large for the MFMA layout's "
                                        "64x-scaled int32 sums");
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (skinny_ok(M, K, N)) {
        // decode batches: the skinny MFMA kernel on the same words
        GemvProblem pb{packed_mfma, magnitude, bias, weight_scale, N, K};
        launch_skinny(pb, q, act_scale, M, y, y_dtype, acc_out, true, st);
        return check_launch("ternary_gemm_mfma");
    }
    GemmProblem pb{packed_mfma, magnitude, bias, weight_scale, N, K};
    launch_gemm_mfma(pb, q, act_scale, M, y, y_dtype, acc_out, st);
    return check_launch("ternary_gemm_mfma");
}

extern "C" int nsosx_find_reserved_code(const uint32_t* packed, int64_t n_codes, int64_t* first_bad,
                                        void* stream) {
    if (!packed || !first_bad || n_codes < 0)
        return fail(NSOSX_ERR_INVALID, "find_reserved_code: bad argument");
    hipStream_t st = static_cast<hipStream_t>(stream);
    unsigned long long* fb = reinterpret_cast<unsigned long long*>(first_bad);
    hipLaunchKernelGGL(fill_u64_kernel, dim3(1), dim3(1), 0, st, fb, ~0ull);
    const int64_t words = (n_codes + 15) / 16;
    if (words > 0) {
        const int blocks = (int)std::min<int64_t>((words + 255) / 256, 4096);
        hipLaunchKernelGGL(find_reserved_kernel, dim3(blocks), dim3(256), 0, st, packed, n_codes, fb);
    }
    hipLaunchKernelGGL(finish_reserved_kernel, dim3(1), dim3(1), 0, st, fb);
    return check_launch("find_reserved_code");
}
