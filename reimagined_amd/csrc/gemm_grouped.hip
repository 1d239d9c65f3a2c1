// The grouped expert GEMMs of the MoE forward on the reference-layout words
// (JambaBlock::forward_moe's per-expert BitLinear loop): one launch over every
// expert's row segment.  The block tiles are in gemm_tiles.hpp.
//
// Reference semantics (OXN/nsos/ of vitorGgC569/reimagined):
//   per-expert GEMMs src/jamba.cpp:3896-3946
//   GEMM + affine    src/bitnet_adapter_avx2.cpp:52-158
#include "gemm_tiles.hpp"

namespace nsosx {

template <int YDT, bool GATHER, bool SQRELU>
__global__ __launch_bounds__(kGemm3Threads, 2) void grouped_gemm3_kernel(
    const nsosx_linear_view* views, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ perm, const int8_t* __restrict__ q,
    const float* __restrict__ act_scale, void* y, int ntn, int ntm, int experts, int compact) {
    extern __shared__ __align__(16) char smem3[];
    // 1-D grid over (n tile, row tile), n fastest; xcd_tile() hands each XCD a
    // contiguous run, so the n tiles of one (expert, m tile) share its rows in one L2.
    // compact: the row tiles are the experts' real tiles in expert order (ntm is an
    // upper bound on their count, sum ceil(rows_e / 128) <= ceil(total / 128) + E),
    // found by walking the offsets; else ntm tiles per expert, most of them empty.
    int nt, rest;
    int e = -1, seg_begin = 0, seg_rows = 0, m0 = 0;
    if (compact) {
        if (!grouped_tile(offsets, experts, ntn, blockIdx.x, nt, e, seg_begin, seg_rows, m0))
            return;
    } else {
        xcd_tile(blockIdx.x, ntn, ntm * experts, nt, rest);
        e = rest / ntm;
        seg_begin = offsets[e];
        seg_rows = offsets[e + 1] - seg_begin;
        m0 = (rest % ntm) * kG3BM;
    }
    if (m0 >= seg_rows) return;
    const nsosx_linear_view v = views[e];
    const int n0 = nt * kG3BN;
    if (n0 >= v.outputs) return;
    GemmProblem pb{v.packed, v.magnitude, v.bias, v.weight_scale, v.outputs, v.inputs};
    gemm3_tile_rows<YDT, GATHER, SQRELU, false>(pb, q, act_scale, perm, seg_begin, seg_rows, n0, m0,
                                                y, smem3);
}

template <int YDT, bool GATHER, bool SQRELU>
__global__ __launch_bounds__(kGemm2Threads) void grouped_gemm2_kernel(const nsosx_linear_view* views,
                                                            const int32_t* __restrict__ offsets,
                                                            const int32_t* __restrict__ perm,
                                                            const int8_t* __restrict__ q,
                                                            const float* __restrict__ act_scale,
                                                            void* y) {
    extern __shared__ __align__(16) char smem2[];
    const int e = blockIdx.z;
    const int seg_begin = offsets[e];
    const int seg_rows = offsets[e + 1] - seg_begin;
    const int m0 = blockIdx.y * kBM2;
    if (m0 >= seg_rows) return;
    const nsosx_linear_view v = views[e];
    const int n0 = blockIdx.x * kBN2;
    if (n0 >= v.outputs) return;
    GemmProblem pb{v.packed, v.magnitude, v.bias, v.weight_scale, v.outputs, v.inputs};
    gemm2_tile<YDT, false, GATHER, SQRELU>(pb, q, act_scale, perm, seg_begin, seg_rows, n0, m0, y,
                                           nullptr, smem2);
}

template <int YDT, bool GATHER, bool SQRELU>
__global__ __launch_bounds__(256) void grouped_gemm_kernel(const nsosx_linear_view* views,
                                                           const int32_t* __restrict__ offsets,
                                                           const int32_t* __restrict__ perm,
                                                           const int8_t* __restrict__ q,
                                                           const float* __restrict__ act_scale,
                                                           void* y) {
    __shared__ __align__(16) char smem[kGemmSmem];
    const int e = blockIdx.z;
    const int seg_begin = offsets[e];
    const int seg_rows = offsets[e + 1] - seg_begin;
    const int m0 = blockIdx.y * kBM;
    if (m0 >= seg_rows) return;
    const nsosx_linear_view v = views[e];
    const int n0 = blockIdx.x * kBN;
    if (n0 >= v.outputs) return;
    GemmProblem pb{v.packed, v.magnitude, v.bias, v.weight_scale, v.outputs, v.inputs};
    gemm_tile<YDT, false, GATHER, SQRELU>(pb, q, act_scale, perm, seg_begin, seg_rows, n0, m0, y,
                                          nullptr, smem);
}

}  // namespace nsosx

using namespace nsosx;

extern "C" int nsosx_grouped_ternary_gemm(const nsosx_linear_view* views_dev, int experts,
                                          const int32_t* offsets, const int32_t* perm, int gather,
                                          const int8_t* q, const float* act_scale, int K, int N,
                                          int max_rows_per_expert, int total_rows,
                                          int squared_relu, void* y, int y_dtype, void* stream) {
    if (!views_dev || !offsets || !q || !act_scale || !y || (gather && !perm))
        return fail(NSOSX_ERR_INVALID, "grouped_ternary_gemm: null pointer");
    if (experts <= 0 || experts > 65535 || K <= 0 || K % 16 || N <= 0 || max_rows_per_expert < 0 ||
        total_rows < 0)
        return fail(NSOSX_ERR_INVALID, "grouped_ternary_gemm: bad shape");
    if (!valid_dtype(y_dtype)) return fail(NSOSX_ERR_INVALID, "grouped_ternary_gemm: bad dtype");
    if (max_rows_per_expert == 0) return NSOSX_OK;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid2((N + kBN2 - 1) / kBN2, (max_rows_per_expert + kBM2 - 1) / kBM2, experts);
    const int ntn3 = (N + kG3BN - 1) / kG3BN;
    // with the total row count the grid covers only the real row tiles (found on the
    // device from the offsets); without it, every expert gets max_rows_per_expert rows
    const int compact = total_rows > 0 && experts <= 1024 ? 1 : 0;
    const int ntm3 = compact ? (total_rows + kG3BM - 1) / kG3BM + experts
                             : (max_rows_per_expert + kG3BM - 1) / kG3BM;
    if ((int64_t)ntn3 * ntm3 * (compact ? 1 : experts) > 0x7fffffff)
        return fail(NSOSX_ERR_INVALID, "grouped_ternary_gemm: too many tiles for one launch");
    const dim3 grid3(ntn3 * ntm3 * (compact ? 1 : experts));
#define NSOSX_GGEMM(YDT, G, S)                                                                  \
    if (K % kG3BK == 0)                                                                         \
        hipLaunchKernelGGL((grouped_gemm3_kernel<YDT, G, S>), grid3, dim3(kGemm3Threads),        \
                           kGemm3Smem, st, views_dev, offsets, perm, q, act_scale, y, ntn3,     \
                           ntm3, experts, compact);                                             \
    else                                                                                        \
        hipLaunchKernelGGL((grouped_gemm2_kernel<YDT, G, S>), grid2, dim3(kGemm2Threads),        \
                           kGemm2Smem, st, views_dev, offsets, perm, q, act_scale, y);
    if (y_dtype == NSOSX_F32) {
        if (gather) { if (squared_relu) { NSOSX_GGEMM(NSOSX_F32, true, true) } else { NSOSX_GGEMM(NSOSX_F32, true, false) } }
        else { if (squared_relu) { NSOSX_GGEMM(NSOSX_F32, false, true) } else { NSOSX_GGEMM(NSOSX_F32, false, false) } }
    } else {
        if (gather) { if (squared_relu) { NSOSX_GGEMM(NSOSX_BF16, true, true) } else { NSOSX_GGEMM(NSOSX_BF16, true, false) } }
        else { if (squared_relu) { NSOSX_GGEMM(NSOSX_BF16, false, true) } else { NSOSX_GGEMM(NSOSX_BF16, false, false) } }
    }
#undef NSOSX_GGEMM
    return check_launch("grouped_ternary_gemm");
}
