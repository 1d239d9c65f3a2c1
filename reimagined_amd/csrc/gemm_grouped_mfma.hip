// The grouped expert GEMMs of the MoE forward on MFMA-layout words
// (nsosx_pack_mfma_layout): one launch over the experts' real row tiles.  The block
// tiles are in gemm_tiles.hpp.
//
// Reference semantics (OXN/nsos/ of vitorGgC569/reimagined):
//   per-expert GEMMs src/jamba.cpp:3896-3946
//   GEMM + affine    src/bitnet_adapter_avx2.cpp:52-158
#include "gemm_tiles.hpp"

#include <atomic>

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

// Split-K tail.  A launch of T tiles on W resident workgroups (2 per CU) runs
// floor(T / W) full rounds and a last round of rem = T mod W tiles; when that round
// would be at most a quarter full (the config-5 down GEMM: 16 of 512) and the tiles are
// long (K of at least kSplitMinKT stages), its tiles are each split over S workgroups
// along K instead (S a power of two <= 8 and <= W / rem, at least 4 k-stages each).  A
// split writes its raw int32 partial sums to the workspace; grouped_gemm3_fixup_kernel,
// launched after, adds a tile's S partials in split order (integer sums: the same bits
// as one workgroup's) and applies the epilogue's dequantization.
constexpr int kSplitMinKT = 16;
struct GroupedTail {
    int main;    // tiles computed whole: 0 .. main - 1
    int rem;     // tail tiles main .. main + rem - 1, split
    int splits;  // 1: no split
};

__device__ __forceinline__ GroupedTail grouped_tail_plan(const int32_t* __restrict__ offsets,
                                                         int experts, int ntn, int W, int KT) {
    int full = 0, part = 0;
    for (int j = 0; j < experts; ++j) {
        const int r = max(offsets[j + 1] - offsets[j], 0);
        full += r / kG3BM;
        part += (r % kG3BM) != 0;
    }
    const int total = ntn * (full + part);
    const int rounds = total / W;
    const int rem = total - rounds * W;
    int splits = 1;
    if (rounds >= 1 && rem > 0 && 4 * rem <= W && KT >= kSplitMinKT)
        while (splits < 8 && 2 * splits * rem <= W && KT % (2 * splits) == 0 &&
               KT / (2 * splits) >= 4)
            splits *= 2;
    GroupedTail t;
    t.splits = splits;
    t.main = splits > 1 ? rounds * W : total;
    t.rem = splits > 1 ? rem : 0;
    return t;
}

template <int YDT, bool GATHER, bool SQRELU>
__global__ __launch_bounds__(kGemm3Threads, 2) void grouped_gemm3_mfma_split_kernel(
    const nsosx_linear_view* views, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ perm, const int8_t* __restrict__ q,
    const float* __restrict__ act_scale, void* y, int ntn, int experts, int W, int KT,
    int32_t* __restrict__ raw) {
    extern __shared__ __align__(16) char smem4[];
    const GroupedTail plan = grouped_tail_plan(offsets, experts, ntn, W, KT);
    const int L = blockIdx.x;
    int tile = L, kt0 = 0, kt1 = -1;
    int32_t* out_raw = nullptr;
    if (L >= plan.main) {
        const int u = L - plan.main;
        if (u >= plan.rem * plan.splits) return;
        tile = plan.main + u / plan.splits;
        const int per = KT / plan.splits;
        kt0 = (u % plan.splits) * per;
        kt1 = kt0 + per;
        out_raw = raw + (int64_t)u * kG3TileInts;
    }
    int nt, e = -1, seg_begin = 0, seg_rows = 0, m0 = 0;
    if (!grouped_tile(offsets, experts, ntn, tile, nt, e, seg_begin, seg_rows, m0)) return;
    if (m0 >= seg_rows) return;
    const nsosx_linear_view v = views[e];
    const int n0 = nt * kG3BN;
    if (n0 >= v.outputs) return;
    GemmProblem pb{v.packed, v.magnitude, v.bias, v.weight_scale, v.outputs, v.inputs};
    gemm3_tile_rows<YDT, GATHER, SQRELU, true>(pb, q, act_scale, perm, seg_begin, seg_rows, n0, m0,
                                               y, smem4, kt0, kt1, out_raw);
}

// The tail's fixup, element-wise so that many CUs share the partials' reads (one
// workgroup per part: fewer, each reading several parts, measured slower): 32
// workgroups per split tile; in part j thread t owns
// int4 j of producer thread t in the raw layout (gemm3_store_raw), i.e. accumulators
// acc[a][b][4c .. 4c + 3] with j = 16 a + 4 b + c: token m0 + 32 b + (t & 31), outputs
// n0 + 64 (t >> 6) + 4 ((t >> 5) & 1) + 32 a + 8 c + 0..3 (gemm3_epilogue's map).  The
// dequantization is gemm3_epilogue's (dequant, then the squared ReLU), per element.
constexpr int kFixupParts = 32;  // 8192 int4 per tile / 256 threads
constexpr int kFixupWgs = 32;    // workgroups per split tile

template <int YDT, bool GATHER, bool SQRELU>
__global__ __launch_bounds__(kGemm3Threads) void grouped_gemm3_fixup_kernel(
    const nsosx_linear_view* views, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ perm, const float* __restrict__ act_scale, void* y, int ntn,
    int experts, int W, int KT, const int32_t* __restrict__ raw) {
    const GroupedTail plan = grouped_tail_plan(offsets, experts, ntn, W, KT);
    const int i = blockIdx.x / kFixupWgs;
    if (i >= plan.rem) return;  // also every workgroup when nothing was split
    int nt, e = -1, seg_begin = 0, seg_rows = 0, m0 = 0;
    if (!grouped_tile(offsets, experts, ntn, plan.main + i, nt, e, seg_begin, seg_rows, m0))
        return;
    if (m0 >= seg_rows) return;
    const nsosx_linear_view v = views[e];
    const int n0 = nt * kG3BN;
    if (n0 >= v.outputs) return;
    const int t = threadIdx.x;
    for (int j = blockIdx.x % kFixupWgs; j < kFixupParts; j += kFixupWgs) {
        const int a = j >> 4, b = (j >> 2) & 3, c = j & 3;
        const int ml = m0 + 32 * b + (t & 31);
        if (ml >= seg_rows) continue;  // (the rows of partial tiles' empty 32-row blocks)
        int4 sum = make_int4(0, 0, 0, 0);
        const int64_t at = (int64_t)(j * kGemm3Threads + t) * 4;
        for (int sp = 0; sp < plan.splits; ++sp) {
            const int4 p = *reinterpret_cast<const int4*>(raw + ((int64_t)i * plan.splits + sp) *
                                                                     kG3TileInts + at);
            sum.x += p.x; sum.y += p.y; sum.z += p.z; sum.w += p.w;
        }
        // MFMA-layout operands carry 64 x the ternary values: every partial is a multiple of
        // 64, so shifting the sum equals shifting one workgroup's accumulators
        const int accs[4] = {sum.x >> 6, sum.y >> 6, sum.z >> 6, sum.w >> 6};
        const int64_t orow = seg_begin + ml;
        const int arow = GATHER ? perm[orow] : (int)orow;
        const float comb = __fmul_rn(act_scale[arow], v.weight_scale);
        const int nb = n0 + 64 * (t >> 6) + 4 * ((t >> 5) & 1) + 32 * a + 8 * c;
        float val[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int n = min(nb + r, v.outputs - 1);  // columns past N are never stored
            val[r] = dequant(accs[r], comb, v.magnitude, v.bias, n);
            if (SQRELU) {
                val[r] = val[r] > 0.0f ? val[r] : 0.0f;
                val[r] = __fmul_rn(val[r], val[r]);
            }
        }
        const int64_t o = orow * v.outputs + nb;
        if (nb + 3 < v.outputs && (o & 3) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0) {
            // the four outputs as one 16-byte (f32) or 8-byte (bf16) store
            if constexpr (YDT == NSOSX_F32)
                *reinterpret_cast<float4*>(static_cast<float*>(y) + o) =
                    make_float4(val[0], val[1], val[2], val[3]);
            else
                *reinterpret_cast<uint2*>(static_cast<uint16_t*>(y) + o) =
                    make_uint2(pack_bf16x2(val[0], val[1]), pack_bf16x2(val[2], val[3]));
        } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (nb + r < v.outputs) store_act<YDT>(y, o + r, val[r]);
        }
    }
}

// Workgroups resident at once on the current device for the 256 x 128 tile kernels
// (2 per CU), looked up once per device.
static int gemm3_resident_wgs() {
    constexpr int kMaxDev = 64;
    static std::atomic<int> cached[kMaxDev];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
    if (dev < kMaxDev) {
        const int w = cached[dev].load(std::memory_order_relaxed);
        if (w > 0) return w;
    }
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
        return 0;
    if (dev < kMaxDev) cached[dev].store(2 * cus, std::memory_order_relaxed);
    return 2 * cus;
}

}  // namespace nsosx

using namespace nsosx;

extern "C" int64_t nsosx_grouped_ternary_gemm_mfma_workspace(void) {
    const int W = gemm3_resident_wgs();
    return W > 0 ? (int64_t)W * kG3TileInts * 4 : -1;
}

extern "C" int nsosx_grouped_ternary_gemm_mfma_ws(const nsosx_linear_view* views_dev, int experts,
                                                  const int32_t* offsets, const int32_t* perm,
                                                  int gather, const int8_t* q,
                                                  const float* act_scale, int K, int N,
                                                  int total_rows, int squared_relu, void* y,
                                                  int y_dtype, void* workspace,
                                                  int64_t workspace_bytes, void* stream) {
    if (!views_dev || !offsets || !q || !act_scale || !y || !workspace || (gather && !perm))
        return fail(NSOSX_ERR_INVALID, "grouped_ternary_gemm_mfma_ws: null pointer");
    if (experts <= 0 || experts > 1024 || K <= 0 || K % kG3BK || N <= 0 || total_rows <= 0)
        return fail(NSOSX_ERR_INVALID,
                    "grouped_ternary_gemm_mfma_ws: bad shape (K % 128 == 0, <= 1024 experts, "
                    "total_rows > 0: offsets[experts] or an upper bound)");
    if (K > kMfmaLayoutMaxK)
        return fail(NSOSX_ERR_OVERFLOW, "grouped_ternary_gemm_mfma_ws: K too large for the MFMA "
                                        "layout's 64x-scaled int32 sums");
    if (!valid_dtype(y_dtype))
        return fail(NSOSX_ERR_INVALID, "grouped_ternary_gemm_mfma_ws: bad dtype");
    const int W = gemm3_resident_wgs();
    if (W <= 0) return fail(NSOSX_ERR_LAUNCH, "grouped_ternary_gemm_mfma_ws: no device");
    if (workspace_bytes < (int64_t)W * kG3TileInts * 4 ||
        (reinterpret_cast<uintptr_t>(workspace) & 15) != 0)
        return fail(NSOSX_ERR_INVALID,
                    "grouped_ternary_gemm_mfma_ws: workspace below "
                    "nsosx_grouped_ternary_gemm_mfma_workspace() bytes or not 16-byte aligned");
    const int ntn = (N + kG3BN - 1) / kG3BN;
    const int ntm = (total_rows + kG3BM - 1) / kG3BM + experts;
    // whole tiles (at most ntn * ntm) and the splits of a tail (at most W)
    if ((int64_t)ntn * ntm + W > 0x7fffffff)
        return fail(NSOSX_ERR_INVALID, "grouped_ternary_gemm_mfma_ws: too many tiles");
    const int KT = K / kG3BK;
    // tiles too short to split: the whole-tile launch alone
    if (KT < kSplitMinKT)
        return nsosx_grouped_ternary_gemm_mfma(views_dev, experts, offsets, perm, gather, q,
                                               act_scale, K, N, total_rows, squared_relu, y,
                                               y_dtype, stream);
    hipStream_t st = static_cast<hipStream_t>(stream);
    int32_t* raw = static_cast<int32_t*>(workspace);
#define NSOSX_GGS(YDT, G, S)                                                                     \
    hipLaunchKernelGGL((grouped_gemm3_mfma_split_kernel<YDT, G, S>), dim3(ntn * ntm + W),        \
                       dim3(kGemm3Threads), kGemm3Smem, st, views_dev, offsets, perm, q,         \
                       act_scale, y, ntn, experts, W, KT, raw);                                  \
    hipLaunchKernelGGL((grouped_gemm3_fixup_kernel<YDT, G, S>), dim3(W / 4 * kFixupWgs),      \
                       dim3(kGemm3Threads), 0, st, views_dev, offsets, perm, act_scale, y, ntn,  \
                       experts, W, KT, raw);
    if (y_dtype == NSOSX_F32) {
        if (gather) { if (squared_relu) { NSOSX_GGS(NSOSX_F32, true, true) } else { NSOSX_GGS(NSOSX_F32, true, false) } }
        else { if (squared_relu) { NSOSX_GGS(NSOSX_F32, false, true) } else { NSOSX_GGS(NSOSX_F32, false, false) } }
    } else {
        if (gather) { if (squared_relu) { NSOSX_GGS(NSOSX_BF16, true, true) } else { NSOSX_GGS(NSOSX_BF16, true, false) } }
        else { if (squared_relu) { NSOSX_GGS(NSOSX_BF16, false, true) } else { NSOSX_GGS(NSOSX_BF16, false, false) } }
    }
#undef NSOSX_GGS
    return check_launch("grouped_ternary_gemm_mfma_ws");
}

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
