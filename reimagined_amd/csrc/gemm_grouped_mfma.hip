// The grouped expert GEMMs of the MoE forward on MFMA-layout words
// (nsosx_pack_mfma_layout): one launch over the experts' real row tiles.  The block
// tiles are in gemm_tiles.hpp.
//
// Reference semantics (OXN/nsos/ of vitorGgC569/reimagined):
//   per-expert GEMMs src/jamba.cpp:3896-3946
//   GEMM + affine    src/bitnet_adapter_avx2.cpp:52-158
#include "gemm_tiles.hpp"

namespace nsosx {

template <int YDT, bool GATHER, bool SQRELU>
__global__ __launch_bounds__(kGemm3Threads, 2) void grouped_gemm3_mfma_kernel(
    const nsosx_linear_view* views, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ perm, const int8_t* __restrict__ q,
    const float* __restrict__ act_scale, void* y, int ntn, int ntm, int experts) {
    extern __shared__ __align__(16) char smem4[];
    // compact row tiles, as grouped_gemm3_kernel's
    int nt, e = -1, seg_begin = 0, seg_rows = 0, m0 = 0;
    if (!grouped_tile(offsets, experts, ntn, blockIdx.x, nt, e, seg_begin, seg_rows, m0)) return;
    if (m0 >= seg_rows) return;
    const nsosx_linear_view v = views[e];
    const int n0 = nt * kG3BN;
    if (n0 >= v.outputs) return;
    GemmProblem pb{v.packed, v.magnitude, v.bias, v.weight_scale, v.outputs, v.inputs};
    gemm3_tile_rows<YDT, GATHER, SQRELU, true>(pb, q, act_scale, perm, seg_begin, seg_rows, n0, m0,
                                               y, smem4);
}

}  // namespace nsosx

using namespace nsosx;

extern "C" int nsosx_grouped_ternary_gemm_mfma(const nsosx_linear_view* views_dev, int experts,
                                               const int32_t* offsets, const int32_t* perm,
                                               int gather, const int8_t* q,
                                               const float* act_scale, int K, int N,
                                               int total_rows, int squared_relu, void* y,
                                               int y_dtype, void* stream) {
    if (!views_dev || !offsets || !q || !act_scale || !y || (gather && !perm))
        return fail(NSOSX_ERR_INVALID, "grouped_ternary_gemm_mfma: null pointer");
    // total_rows sizes the launch (there is no per-expert bound to fall back on, as
    // nsosx_grouped_ternary_gemm's max_rows_per_expert): it must be given, > 0
    if (experts <= 0 || experts > 1024 || K <= 0 || K % kG3BK || N <= 0 || total_rows <= 0)
        return fail(NSOSX_ERR_INVALID,
                    "grouped_ternary_gemm_mfma: bad shape (K % 128 == 0, <= 1024 experts, "
                    "total_rows > 0: offsets[experts] or an upper bound)");
    if (K > kMfmaLayoutMaxK)
        return fail(NSOSX_ERR_OVERFLOW, "grouped_ternary_gemm_mfma: K too large for the MFMA "
                                        "layout's 64x-scaled int32 sums");
    if (!valid_dtype(y_dtype))
        return fail(NSOSX_ERR_INVALID, "grouped_ternary_gemm_mfma: bad dtype");
    const int ntn = (N + kG3BN - 1) / kG3BN;
    const int ntm = (total_rows + kG3BM - 1) / kG3BM + experts;
    if ((int64_t)ntn * ntm > 0x7fffffff)
        return fail(NSOSX_ERR_INVALID, "grouped_ternary_gemm_mfma: too many tiles");
    hipStream_t st = static_cast<hipStream_t>(stream);
#define NSOSX_GGM(YDT, G, S)                                                                     \
    hipLaunchKernelGGL((grouped_gemm3_mfma_kernel<YDT, G, S>), dim3(ntn * ntm), dim3(kGemm3Threads),   \
                       kGemm3Smem, st, views_dev, offsets, perm, q, act_scale, y, ntn, ntm,       \
                       experts);
    if (y_dtype == NSOSX_F32) {
        if (gather) { if (squared_relu) { NSOSX_GGM(NSOSX_F32, true, true) } else { NSOSX_GGM(NSOSX_F32, true, false) } }
        else { if (squared_relu) { NSOSX_GGM(NSOSX_F32, false, true) } else { NSOSX_GGM(NSOSX_F32, false, false) } }
    } else {
        if (gather) { if (squared_relu) { NSOSX_GGM(NSOSX_BF16, true, true) } else { NSOSX_GGM(NSOSX_BF16, true, false) } }
        else { if (squared_relu) { NSOSX_GGM(NSOSX_BF16, false, true) } else { NSOSX_GGM(NSOSX_BF16, false, false) } }
    }
#undef NSOSX_GGM
    return check_launch("grouped_ternary_gemm_mfma");
}
