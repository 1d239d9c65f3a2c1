// Device-side weight statistics over the packed ternary format.
//
// compute_weight_row_sums (OXN/nsos/src/bitlinear.cpp:36-73) sums each row of
// the unpacked int8 weights when BitLinear repacks: sum_k w[n, k] in int32.
// Here it runs on the packed words already resident on the device, one wave
// per row: a word's 16 codes contribute (#code 2) - (#code 0), which two
// population counts give without unpacking (codes 1 and the reserved 3 decode
// to 0, src/bitnet_adapter.cpp:31).
#include "common.hpp"

namespace nsosx {

__global__ __launch_bounds__(256) void row_sums_kernel(const uint32_t* __restrict__ packed,
                                                       int N, int words_per_row,
                                                       int32_t* __restrict__ sums) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= N) return;
    const uint32_t* src = packed + (int64_t)row * words_per_row;
    int acc = 0;
    for (int i = lane; i < words_per_row; i += 64) {
        const uint32_t w = src[i];
        const uint32_t lo = w & 0x55555555u;          // bit 0 of each code
        const uint32_t hi = (w >> 1) & 0x55555555u;   // bit 1 of each code
        acc += __popc(hi & ~lo) - __popc(~hi & ~lo & 0x55555555u);
    }
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
    if (lane == 0) sums[row] = acc;
}

}  // namespace nsosx

using namespace nsosx;

extern "C" int nsosx_weight_row_sums(const uint32_t* packed, int N, int K, int32_t* sums,
                                     void* stream) {
    if (!packed || !sums) return fail(NSOSX_ERR_INVALID, "weight_row_sums: null pointer");
    if (N <= 0 || K <= 0 || K % 16 != 0)
        return fail(NSOSX_ERR_INVALID,
                    "weight_row_sums: need N > 0 and K a positive multiple of 16");
    const dim3 grid((N + 3) / 4);
    hipLaunchKernelGGL(row_sums_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                       packed, N, K / 16, sums);
    return check_launch("weight_row_sums");
}
