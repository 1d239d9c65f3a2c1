// BitLinear prefill GEMMs on gfx950's int8 MFMA: the dense GEMM on the
// reference words and on the MFMA layout, and the upload-time repack into the
// MFMA layout.  The block tiles are in gemm_tiles.hpp.
//
// Reference semantics (OXN/nsos/ of vitorGgC569/reimagined):
//   GEMM + affine src/bitnet_adapter_avx2.cpp:52-158
//   packed format src/bitnet_adapter.cpp:570-606
#include "gemm_tiles.hpp"

namespace nsosx {

template <int YDT, bool ACC_OUT>
__global__ __launch_bounds__(kGemm2Threads) void gemm2_kernel(GemmProblem pb, const int8_t* __restrict__ q,
                                                    const float* __restrict__ act_scale, int M,
                                                    void* y, int32_t* acc_out) {
    extern __shared__ __align__(16) char smem2[];
    const int ntn = (pb.N + kBN2 - 1) / kBN2;
    const int ntm = (M + kBM2 - 1) / kBM2;
    int nt, mt;
    xcd_tile(blockIdx.x, ntn, ntm, nt, mt);
    gemm2_tile<YDT, ACC_OUT, false, false>(pb, q, act_scale, nullptr, 0, M, nt * kBN2, mt * kBM2,
                                           y, acc_out, smem2);
}

template <int YDT, bool ACC_OUT>
__global__ __launch_bounds__(kGemm3Threads, 2) void gemm3_kernel(GemmProblem pb,
                                                                 const int8_t* __restrict__ q,
                                                                 const float* __restrict__ act_scale,
                                                                 int M, void* y, int32_t* acc_out) {
    extern __shared__ __align__(16) char smem3[];
    const int ntn = (pb.N + kG3BN - 1) / kG3BN;
    const int ntm = (M + kG3BM - 1) / kG3BM;
    int nt, mt;
    xcd_tile(blockIdx.x, ntn, ntm, nt, mt);
    gemm3_tile<YDT, ACC_OUT, false, false>(pb, q, act_scale, nullptr, 0, M, nt * kG3BN,
                                           mt * kG3BM, y, acc_out, smem3);
}

// ===========================================================================
// The prefill GEMM on weights repacked into the MFMA layout
// (nsosx_pack_mfma_layout): inside each 16-code word, code k is the two's-
// complement ternary value at bits 8 (k % 4) + 6 - 2 (k / 4) (the reserved code
// 3 is stored as 0).  A word then unpacks with one shift and one mask per output
// dword straight into natural k order, each byte 64 x its value; the reference
// layout needs a table lookup per dword and a further 4x4 byte transpose per
// word.  gemm3's block, ring and loads otherwise.
// ===========================================================================
template <int YDT, bool ACC_OUT>
__global__ __launch_bounds__(kGemm3Threads, 2) void gemm3_mfma_kernel(GemmProblem pb,
                                                                 const int8_t* __restrict__ q,
                                                                 const float* __restrict__ act_scale,
                                                                 int M, void* y, int32_t* acc_out) {
    extern __shared__ __align__(16) char smem4[];
    const int ntn = (pb.N + kG3BN - 1) / kG3BN;
    const int ntm = (M + kG3BM - 1) / kG3BM;
    int nt, mt;
    xcd_tile(blockIdx.x, ntn, ntm, nt, mt);
    gemm3_tile<YDT, ACC_OUT, false, false, true>(pb, q, act_scale, nullptr, 0, M, nt * kG3BN,
                                                 mt * kG3BM, y, acc_out, smem4);
}

// Reference layout -> MFMA layout, word by word: code k (-1 / 0 / +1 / reserved 0
// for 0 / 1 / 2 / 3) becomes the two's-complement field (3 / 0 / 1 / 0) at bits
// 8 (k % 4) + 6 - 2 (k / 4), the layout unpack_word_mfma() reads.
__global__ __launch_bounds__(256) void pack_mfma_kernel(const uint32_t* __restrict__ src,
                                                        int64_t n, uint32_t* __restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const uint32_t w = src[i];
    uint32_t o = 0;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const uint32_t f = (0x0103u >> (4 * ((w >> (2 * k)) & 3u))) & 3u;
        o |= f << (8 * (k & 3) + 6 - 2 * (k >> 2));
    }
    dst[i] = o;
}

template <int YDT, bool ACC_OUT>
__global__ __launch_bounds__(256) void gemm_kernel(GemmProblem pb, const int8_t* __restrict__ q,
                                                   const float* __restrict__ act_scale, int M,
                                                   void* y, int32_t* acc_out) {
    __shared__ __align__(16) char smem[kGemmSmem];
    const int n0 = blockIdx.x * kBN;
    const int m0 = blockIdx.y * kBM;
    gemm_tile<YDT, ACC_OUT, false, false>(pb, q, act_scale, nullptr, 0, M, n0, m0, y, acc_out,
                                          smem);
}

template <int YDT>
static void launch_gemm_t(const GemmProblem& pb, const int8_t* q, const float* as, int M,
                          void* y, int32_t* acc, hipStream_t st) {
    if (M > kBM) {
        const int tiles = ((pb.N + kBN2 - 1) / kBN2) * ((M + kBM2 - 1) / kBM2);
        if (pb.K % kG3BK == 0) {
            const int tiles3 = ((pb.N + kG3BN - 1) / kG3BN) * ((M + kG3BM - 1) / kG3BM);
            if (acc)
                hipLaunchKernelGGL((gemm3_kernel<YDT, true>), dim3(tiles3), dim3(kGemm3Threads),
                                   kGemm3Smem, st, pb, q, as, M, y, acc);
            else
                hipLaunchKernelGGL((gemm3_kernel<YDT, false>), dim3(tiles3), dim3(kGemm3Threads),
                                   kGemm3Smem, st, pb, q, as, M, y, acc);
            return;
        }
        if (acc)
            hipLaunchKernelGGL((gemm2_kernel<YDT, true>), dim3(tiles), dim3(kGemm2Threads), kGemm2Smem, st,
                               pb, q, as, M, y, acc);
        else
            hipLaunchKernelGGL((gemm2_kernel<YDT, false>), dim3(tiles), dim3(kGemm2Threads), kGemm2Smem, st,
                               pb, q, as, M, y, acc);
        return;
    }
    const dim3 grid((pb.N + kBN - 1) / kBN, (M + kBM - 1) / kBM), block(256);
    if (acc)
        hipLaunchKernelGGL((gemm_kernel<YDT, true>), grid, block, 0, st, pb, q, as, M, y, acc);
    else
        hipLaunchKernelGGL((gemm_kernel<YDT, false>), grid, block, 0, st, pb, q, as, M, y, acc);
}

void launch_gemm(const GemmProblem& pb, const int8_t* q, const float* as, int M, void* y,
                 int y_dtype, int32_t* acc, hipStream_t st) {
    if (y_dtype == NSOSX_F32) launch_gemm_t<NSOSX_F32>(pb, q, as, M, y, acc, st);
    else launch_gemm_t<NSOSX_BF16>(pb, q, as, M, y, acc, st);
}

void launch_gemm_mfma(const GemmProblem& pb, const int8_t* q, const float* as, int M, void* y,
                      int y_dtype, int32_t* acc, hipStream_t st) {
    const int tiles = ((pb.N + kG3BN - 1) / kG3BN) * ((M + kG3BM - 1) / kG3BM);
#define NSOSX_GM(YDT, ACC)                                                                    \
    hipLaunchKernelGGL((gemm3_mfma_kernel<YDT, ACC>), dim3(tiles), dim3(kGemm3Threads), kGemm3Smem, \
                       st, pb, q, as, M, y, acc);
    if (y_dtype == NSOSX_F32) {
        if (acc) { NSOSX_GM(NSOSX_F32, true) } else { NSOSX_GM(NSOSX_F32, false) }
    } else {
        if (acc) { NSOSX_GM(NSOSX_BF16, true) } else { NSOSX_GM(NSOSX_BF16, false) }
    }
#undef NSOSX_GM
}

}  // namespace nsosx

using namespace nsosx;

extern "C" int nsosx_pack_mfma_layout(const uint32_t* packed, int64_t n_words, uint32_t* out,
                                      void* stream) {
    if (!packed || !out || n_words < 0)
        return fail(NSOSX_ERR_INVALID, "pack_mfma_layout: bad argument");
    if (n_words == 0) return NSOSX_OK;
    hipLaunchKernelGGL(pack_mfma_kernel, dim3((unsigned)((n_words + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), packed, n_words, out);
    return check_launch("pack_mfma_layout");
}
