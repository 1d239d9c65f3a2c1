// Top-k MoE routing on gfx950: softmax + top-k + renormalisation per row,
// then the deterministic expert-major, rows-ascending token permutation
// (counts -> exclusive scan -> stable ranks) with no host round trip, and
// the weighted combine in ascending expert order.
//
// Reference semantics (OXN/nsos/ of vitorGgC569/reimagined):
//   softmax           Tensor::softmax, src/tensor.cpp:3428-3450
//   top-k + renorm    MoERouter::forward CPU path, src/jamba.cpp:8268-8297
//   permutation       JambaBlock::forward_moe, src/jamba.cpp:3882-3894
//   combine           src/jamba.cpp:3947-3969
#include "common.hpp"

namespace nsosx {

constexpr int kMaxExperts = 64;
constexpr int kRouteBlock = 256;  // rows per dispatch block

// One thread per row.  The softmax keeps the reference's order of
// operations: running max, exp(x - max), an in-order float sum, one
// multiply by 1/max(sum, 1e-8f).  Top-k is a selection under the strict
// order (value desc, index asc); renormalisation sums the selected values in
// rank order and multiplies by 1/max(sum, 1e-9f).  EMAX (>= E) bounds every
// loop at compile time, so the row's probabilities stay in registers (a
// runtime-indexed array of 64 lives in scratch memory); experts past E are
// masked out.
// A padding row (valid_rows[r] == 0, as launch_moe_zero_invalid_rows_kernel reads the
// mask, src/cuda/moe_kernels.cu:118-125) is absent from routing: its weights are all
// zero (MoERouter::forward zeroes them after the top-k, src/jamba.cpp:8195-8214,
// 8299-8304), its selections are -1, and it takes no dispatch slot (the reference's
// dispatch counts only nonzero weights, src/cuda/moe_kernels.cu:226-235, 305-319).
// Any k <= E (MoERouter::forward's partial sort, src/jamba.cpp:8268-8297).  Returns the
// row's selected experts as a bit mask (0 for a padding row).
template <int EMAX>
__device__ __forceinline__ uint64_t route_one_row(const float* __restrict__ logits,
                                                  const uint8_t* __restrict__ valid_rows, int r,
                                                  int E, int k, float* __restrict__ weights,
                                                  int32_t* __restrict__ selected) {
    if (valid_rows && valid_rows[r] == 0) {
        float* w = weights + (int64_t)r * E;
        for (int j = 0; j < E; ++j) w[j] = 0.0f;
        for (int i = 0; i < k; ++i) selected[(int64_t)r * k + i] = -1;
        return 0;
    }
    const float* src = logits + (int64_t)r * E;
    float p[EMAX];
#pragma unroll
    for (int j = 0; j < EMAX; ++j) p[j] = j < E ? src[j] : 0.0f;
    float mx = p[0];
#pragma unroll
    for (int j = 1; j < EMAX; ++j)
        if (j < E) mx = p[j] > mx ? p[j] : mx;
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < EMAX; ++j)
        if (j < E) {
            p[j] = expf(p[j] - mx);
            sum = sum + p[j];
        }
    const float inv = 1.0f / (sum > 1e-8f ? sum : 1e-8f);
#pragma unroll
    for (int j = 0; j < EMAX; ++j) p[j] = p[j] * inv;
    uint64_t taken = 0;
    float ssum = 0.0f;
    for (int i = 0; i < k; ++i) {
        int best = -1;
        float bv = 0.0f;
#pragma unroll
        for (int j = 0; j < EMAX; ++j) {
            const bool free = j < E && !((taken >> j) & 1ull);
            if (free && (best < 0 || p[j] > bv)) {  // ties keep the lower index
                best = j;
                bv = p[j];
            }
        }
        taken |= 1ull << best;
        selected[(int64_t)r * k + i] = best;
        ssum = ssum + bv;
    }
    // k == E keeps the raw softmax: the reference masks and renormalises only when
    // top_k < num_experts (src/jamba.cpp:8268)
    const float inv2 = 1.0f / (ssum > 1e-9f ? ssum : 1e-9f);
    const bool renorm = k < E;
    float* w = weights + (int64_t)r * E;
#pragma unroll
    for (int j = 0; j < EMAX; ++j)
        if (j < E) w[j] = ((taken >> j) & 1ull) ? (renorm ? p[j] * inv2 : p[j]) : 0.0f;
    return taken;
}

// Row r's selection list as an expert bit mask (-1 entries, padding rows, add nothing),
// with its first min(k, 8) choices kept in registers.
__device__ __forceinline__ uint64_t row_selection(const int32_t* __restrict__ selected, int r,
                                                  int k, int (&first)[8]) {
    uint64_t mask = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        first[i] = i < k ? selected[(int64_t)r * k + i] : -1;
        if (first[i] >= 0) mask |= 1ull << first[i];
    }
    for (int i = 8; i < k; ++i) {
        const int e = selected[(int64_t)r * k + i];
        if (e >= 0) mask |= 1ull << e;
    }
    return mask;
}

// Position of expert e in row r's selection list (e is in it).
__device__ __forceinline__ int choice_of(const int32_t* __restrict__ selected, int r, int k, int e,
                                         const int (&first)[8]) {
    int which = -1;
#pragma unroll
    for (int i = 0; i < 8; ++i)
        if (first[i] == e) which = i;
    if (which < 0)
        for (int i = 8; i < k; ++i)
            if (selected[(int64_t)r * k + i] == e) which = i;
    return which;
}

template <int EMAX>
__global__ __launch_bounds__(256) void route_rows_kernel(const float* __restrict__ logits,
                                                         const uint8_t* __restrict__ valid_rows,
                                                         int rows, int E, int k,
                                                         float* __restrict__ weights,
                                                         int32_t* __restrict__ selected) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r < rows) route_one_row<EMAX>(logits, valid_rows, r, E, k, weights, selected);
}

// Routing fused with the per-block expert counts: one thread per row of a
// dispatch block of kRouteBlock rows, then how many of the block's rows
// selected each expert (LDS counters; counts are order-free).
template <int EMAX>
__global__ __launch_bounds__(256) void route_rows_count_kernel(const float* __restrict__ logits,
                                                               const uint8_t* __restrict__ valid_rows,
                                                               int rows, int E, int k,
                                                               float* __restrict__ weights,
                                                               int32_t* __restrict__ selected,
                                                               int32_t* __restrict__ block_counts) {
    __shared__ int32_t cnt[kMaxExperts];
    const int tid = threadIdx.x;
    if (tid < E) cnt[tid] = 0;
    __syncthreads();
    const int r = blockIdx.x * kRouteBlock + tid;
    if (r < rows)
        for (uint64_t m = route_one_row<EMAX>(logits, valid_rows, r, E, k, weights, selected); m;
             m &= m - 1)
            atomicAdd(&cnt[__builtin_ctzll(m)], 1);
    __syncthreads();
    if (tid < E) block_counts[(int64_t)blockIdx.x * E + tid] = cnt[tid];
}

// Per dispatch block of 256 rows: how many of its rows selected each expert.
__global__ __launch_bounds__(256) void route_count_kernel(const int32_t* __restrict__ selected,
                                                          int rows, int E, int k,
                                                          int32_t* __restrict__ block_counts) {
    __shared__ int32_t cnt[kMaxExperts];
    const int tid = threadIdx.x;
    if (tid < E) cnt[tid] = 0;
    __syncthreads();
    const int r = blockIdx.x * kRouteBlock + tid;
    if (r < rows)
        for (int i = 0; i < k; ++i) {
            const int e = selected[(int64_t)r * k + i];
            if (e >= 0) atomicAdd(&cnt[e], 1);  // -1: a padding row
        }
    __syncthreads();
    if (tid < E) block_counts[(int64_t)blockIdx.x * E + tid] = cnt[tid];
}

// Single workgroup: counts[e], offsets = exclusive scan over experts, and the
// exclusive scan over blocks of each expert's per-block counts (in place).
__global__ __launch_bounds__(64) void route_scan_kernel(int32_t* __restrict__ block_counts,
                                                        int nblocks, int E,
                                                        int32_t* __restrict__ counts,
                                                        int32_t* __restrict__ offsets) {
    __shared__ int32_t tot[kMaxExperts];
    const int e = threadIdx.x;
    if (e < E) {
        int run = 0;
        for (int b = 0; b < nblocks; ++b) {
            const int v = block_counts[(int64_t)b * E + e];
            block_counts[(int64_t)b * E + e] = run;
            run += v;
        }
        tot[e] = run;
        counts[e] = run;
    }
    __syncthreads();
    if (e == 0) {
        int run = 0;
        for (int j = 0; j < E; ++j) {
            offsets[j] = run;
            run += tot[j];
        }
        offsets[E] = run;
    }
}

// Stable ranks: within a block, rows are ranked per expert in ascending row
// order with wave ballots and a prefix over the block's four waves.
__global__ __launch_bounds__(256) void route_assign_kernel(const int32_t* __restrict__ selected,
                                                           int rows, int E, int k,
                                                           const int32_t* __restrict__ block_base,
                                                           const int32_t* __restrict__ offsets,
                                                           int32_t* __restrict__ perm,
                                                           int32_t* __restrict__ slot_of) {
    __shared__ int32_t wave_cnt[4][kMaxExperts];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int r = blockIdx.x * kRouteBlock + tid;
    const bool valid = r < rows;
    int first[8];
    const uint64_t mine = valid ? row_selection(selected, r, k, first) : 0;
    if (valid && mine == 0)  // a padding row: no slots
        for (int i = 0; i < k; ++i) slot_of[(int64_t)r * k + i] = -1;
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int e = 0; e < E; ++e) {
        const uint64_t bal = __ballot((mine >> e) & 1ull);
        if (lane == 0) wave_cnt[wave][e] = __popcll(bal);
    }
    __syncthreads();
    for (int e = 0; e < E; ++e) {
        const bool has = (mine >> e) & 1ull;
        const uint64_t bal = __ballot(has);
        if (has) {
            int before = 0;
            for (int w = 0; w < wave; ++w) before += wave_cnt[w][e];
            const int rank = before + __popcll(bal & lt);
            const int slot = offsets[e] + block_base[(int64_t)blockIdx.x * E + e] + rank;
            perm[slot] = r;
            slot_of[(int64_t)r * k + choice_of(selected, r, k, e, first)] = slot;
        }
    }
}

// The exclusive scans fused into the assignment, for up to kPlaceMaxCounts
// per-block counts (dispatch blocks x experts): every block reads all the counts
// into LDS in one coalesced pass and sums them itself (its own base per expert,
// the totals, the expert offsets), block 0 publishes counts and offsets, then
// the stable ranks as route_assign_kernel.  Same slots.
constexpr int kPlaceMaxCounts = 4096;

__global__ __launch_bounds__(256) void route_place_kernel(const int32_t* __restrict__ selected,
                                                          int rows, int E, int k, int nblocks,
                                                          const int32_t* __restrict__ block_counts,
                                                          int32_t* __restrict__ counts,
                                                          int32_t* __restrict__ offsets,
                                                          int32_t* __restrict__ perm,
                                                          int32_t* __restrict__ slot_of) {
    __shared__ int32_t base[kMaxExperts], tot[kMaxExperts], off[kMaxExperts + 1];
    __shared__ int32_t wave_cnt[4][kMaxExperts];
    __shared__ int32_t s_counts[kPlaceMaxCounts];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i < nblocks * E; i += blockDim.x) s_counts[i] = block_counts[i];
    __syncthreads();
    if (tid < E) {
        int before = 0, all = 0;
        for (int b = 0; b < nblocks; ++b) {
            const int v = s_counts[b * E + tid];
            before += b < (int)blockIdx.x ? v : 0;
            all += v;
        }
        base[tid] = before;
        tot[tid] = all;
    }
    __syncthreads();
    if (tid == 0) {
        int run = 0;
        for (int j = 0; j < E; ++j) {
            off[j] = run;
            run += tot[j];
        }
        off[E] = run;
    }
    __syncthreads();
    if (blockIdx.x == 0) {
        if (tid < E) counts[tid] = tot[tid];
        if (tid <= E) offsets[tid] = off[tid];
    }
    const int r = blockIdx.x * kRouteBlock + tid;
    const bool valid = r < rows;
    int first[8];
    const uint64_t mine = valid ? row_selection(selected, r, k, first) : 0;
    if (valid && mine == 0)  // a padding row: no slots
        for (int i = 0; i < k; ++i) slot_of[(int64_t)r * k + i] = -1;
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int e = 0; e < E; ++e) {
        const uint64_t bal = __ballot((mine >> e) & 1ull);
        if (lane == 0) wave_cnt[wave][e] = __popcll(bal);
    }
    __syncthreads();
    for (int e = 0; e < E; ++e) {
        const bool has = (mine >> e) & 1ull;
        const uint64_t bal = __ballot(has);
        if (has) {
            int before = 0;
            for (int w = 0; w < wave; ++w) before += wave_cnt[w][e];
            const int rank = before + __popcll(bal & lt);
            const int slot = off[e] + base[e] + rank;
            perm[slot] = r;
            slot_of[(int64_t)r * k + choice_of(selected, r, k, e, first)] = slot;
        }
    }
}

// out[r, d] = sum over the row's experts in ascending id order of
// expert_out[slot, d] * w[r, e], starting from 0.
template <int IDT, int ODT>
__global__ __launch_bounds__(256) void combine_kernel(const void* __restrict__ expert_out,
                                                      const int32_t* __restrict__ slot_of,
                                                      const int32_t* __restrict__ selected,
                                                      const float* __restrict__ weights, int rows,
                                                      int E, int k, int dim,
                                                      void* __restrict__ out) {
    const int r = blockIdx.y;
    const int d = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows || d >= dim) return;
    int es[8], ss[8];
    const int kk = k < 8 ? k : 8;
    if (selected[(int64_t)r * k] < 0) {  // a padding row (no experts): zero
        store_act<ODT>(out, (int64_t)r * dim + d, 0.0f);
        return;
    }
    if (k > 8) {  // wide routing: the row's experts in ascending id from its selection mask
        int first[8];
        float acc = 0.0f;
        for (uint64_t m = row_selection(selected, r, k, first); m; m &= m - 1) {
            const int e = __builtin_ctzll(m);
            const int i = choice_of(selected, r, k, e, first);
            const int64_t s = slot_of ? slot_of[(int64_t)r * k + i] : (int64_t)r * k + i;
            acc = acc + __fmul_rn(load_act<IDT>(expert_out, s * dim + d),
                                  weights[(int64_t)r * E + e]);
        }
        store_act<ODT>(out, (int64_t)r * dim + d, acc);
        return;
    }
    for (int i = 0; i < kk; ++i) {
        es[i] = selected[(int64_t)r * k + i];
        ss[i] = slot_of ? slot_of[(int64_t)r * k + i] : r * k + i;
    }
    // insertion sort by expert id (k is tiny)
    for (int i = 1; i < kk; ++i) {
        const int e = es[i], s = ss[i];
        int j = i - 1;
        while (j >= 0 && es[j] > e) { es[j + 1] = es[j]; ss[j + 1] = ss[j]; --j; }
        es[j + 1] = e;
        ss[j + 1] = s;
    }
    float acc = 0.0f;
    for (int i = 0; i < kk; ++i) {
        const float v = load_act<IDT>(expert_out, (int64_t)ss[i] * dim + d);
        acc = acc + __fmul_rn(v, weights[(int64_t)r * E + es[i]]);
    }
    store_act<ODT>(out, (int64_t)r * dim + d, acc);
}

// The same sums with a wave per output row: the row's k (expert, slot, weight)
// triples are wave-uniform (scalar loads, sorted once per wave) and each lane
// takes V consecutive elements per step with one vector load per expert (V = 8:
// 16-byte bf16 loads, V = 4 otherwise).  With k <= 2 the loads of up to four steps
// (a row of 2048 bf16) are issued before any is used.  Needs dim % V == 0 and
// 16-byte (f32, or V = 8) / 8-byte (bf16) aligned rows.
template <int IDT, int V>
__device__ __forceinline__ void combine_load(const void* p, int64_t off, float v[V]) {
    if constexpr (IDT == NSOSX_F32) {
#pragma unroll
        for (int j = 0; j < V; j += 4) {
            const float4 t = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + off + j);
            v[j] = t.x; v[j + 1] = t.y; v[j + 2] = t.z; v[j + 3] = t.w;
        }
    } else if constexpr (V == 8) {
        const uint4 t = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + off);
        const uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[2 * j] = __uint_as_float(w[j] << 16);
            v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
        }
    } else {
        const uint2 t = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + off);
        v[0] = __uint_as_float(t.x << 16); v[1] = __uint_as_float(t.x & 0xffff0000u);
        v[2] = __uint_as_float(t.y << 16); v[3] = __uint_as_float(t.y & 0xffff0000u);
    }
}

template <int ODT, int V>
__device__ __forceinline__ void combine_store(void* p, int64_t o, const float acc[V]) {
    if constexpr (ODT == NSOSX_F32) {
#pragma unroll
        for (int j = 0; j < V; j += 4)
            *reinterpret_cast<float4*>(static_cast<float*>(p) + o + j) =
                make_float4(acc[j], acc[j + 1], acc[j + 2], acc[j + 3]);
    } else if constexpr (V == 8) {
        *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p) + o) =
            make_uint4(pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3]),
                       pack_bf16x2(acc[4], acc[5]), pack_bf16x2(acc[6], acc[7]));
    } else {
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p) + o) =
            make_uint2(pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3]));
    }
}

template <int IDT, int ODT, int V>
__global__ __launch_bounds__(256) void combine_rows_kernel(const void* __restrict__ expert_out,
                                                           const int32_t* __restrict__ slot_of,
                                                           const int32_t* __restrict__ selected,
                                                           const float* __restrict__ weights,
                                                           int rows, int E, int k, int dim,
                                                           void* __restrict__ out) {
    const int r = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    if (r >= rows) return;
    const int lane = threadIdx.x & 63;
    int es[8], ss[8];
    float ws[8];
    const int kk = k < 8 ? k : 8;
    if (selected[(int64_t)r * k] < 0) {  // a padding row (no experts): zero
        float zero[V];
#pragma unroll
        for (int j = 0; j < V; ++j) zero[j] = 0.0f;
        for (int d = V * lane; d < dim; d += V * kWave)
            combine_store<ODT, V>(out, (int64_t)r * dim + d, zero);
        return;
    }
    if (k > 8) {
        // wide routing: lane e holds expert e's slot (-1 if the row did not select it) and
        // weight; the sum walks the selected lanes in ascending id
        int my_slot = -1;
        float my_w = 0.0f;
        if (lane < E) {
            for (int i = 0; i < k; ++i)
                if (selected[(int64_t)r * k + i] == lane)
                    my_slot = slot_of ? slot_of[(int64_t)r * k + i] : r * k + i;
            my_w = weights[(int64_t)r * E + lane];
        }
        const uint64_t has = __ballot(my_slot >= 0);
        for (int d = V * lane; d < dim; d += V * kWave) {
            float acc[V];
#pragma unroll
            for (int j = 0; j < V; ++j) acc[j] = 0.0f;
            for (uint64_t m = has; m; m &= m - 1) {
                const int e = __builtin_ctzll(m);
                const int64_t sl = __builtin_amdgcn_readlane(my_slot, e);
                const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_w), e));
                float v[V];
                combine_load<IDT, V>(expert_out, sl * dim + d, v);
#pragma unroll
                for (int j = 0; j < V; ++j) acc[j] = acc[j] + __fmul_rn(v[j], w);
            }
            combine_store<ODT, V>(out, (int64_t)r * dim + d, acc);
        }
        return;
    }
    for (int i = 0; i < kk; ++i) {
        es[i] = selected[(int64_t)r * k + i];
        ss[i] = slot_of ? slot_of[(int64_t)r * k + i] : r * k + i;
    }
    for (int i = 1; i < kk; ++i) {
        const int e = es[i], sl = ss[i];
        int j = i - 1;
        while (j >= 0 && es[j] > e) { es[j + 1] = es[j]; ss[j + 1] = ss[j]; --j; }
        es[j + 1] = e;
        ss[j + 1] = sl;
    }
    for (int i = 0; i < kk; ++i) ws[i] = weights[(int64_t)r * E + es[i]];
    const int64_t orow = (int64_t)r * dim;
    constexpr int S = 4;  // steps whose loads go out together (k <= 2)
    if (kk <= 2) {
        // a missing second expert re-reads the first with weight 0 (never added)
        const int64_t b0 = (int64_t)ss[0] * dim, b1 = (int64_t)ss[kk - 1] * dim;
        for (int d0 = V * lane; d0 < dim; d0 += S * V * kWave) {
            float v0[S][V], v1[S][V];
#pragma unroll
            for (int u = 0; u < S; ++u) {
                const int d = min(d0 + u * V * kWave, dim - V);
                combine_load<IDT, V>(expert_out, b0 + d, v0[u]);
                combine_load<IDT, V>(expert_out, b1 + d, v1[u]);
            }
#pragma unroll
            for (int u = 0; u < S; ++u) {
                const int d = d0 + u * V * kWave;
                if (d >= dim) break;
                float acc[V];
#pragma unroll
                for (int j = 0; j < V; ++j) {
                    acc[j] = 0.0f + __fmul_rn(v0[u][j], ws[0]);
                    if (kk == 2) acc[j] = acc[j] + __fmul_rn(v1[u][j], ws[1]);
                }
                combine_store<ODT, V>(out, orow + d, acc);
            }
        }
        return;
    }
    for (int d = V * lane; d < dim; d += V * kWave) {
        float acc[V];
#pragma unroll
        for (int j = 0; j < V; ++j) acc[j] = 0.0f;
        for (int i = 0; i < kk; ++i) {
            float v[V];
            combine_load<IDT, V>(expert_out, (int64_t)ss[i] * dim + d, v);
#pragma unroll
            for (int j = 0; j < V; ++j) acc[j] = acc[j] + __fmul_rn(v[j], ws[i]);
        }
        combine_store<ODT, V>(out, orow + d, acc);
    }
}

// Per-expert loads: loads[e] = the sum over rows, in ascending row order, of
// weights[r, e] (MoERouter::forward's expert_loads, src/jamba.cpp:8299-8307, the
// order of launch_moe_load_ordered_kernel, src/cuda/moe_kernels.cu:108-116; padding
// rows add their zero weights).  A wave per expert: each lane holds 64 consecutive
// rows' values at a time and lane 0 adds them in order, so the loads of the next
// 64 rows are in flight while the sum runs.
__global__ __launch_bounds__(64) void route_loads_kernel(const float* __restrict__ weights,
                                                         int rows, int E,
                                                         float* __restrict__ loads) {
    const int e = blockIdx.x;
    const int lane = threadIdx.x;
    __shared__ float s_v[2][kWave];
    float total = 0.0f;
    int buf = 0;
    float v = lane < rows ? weights[(int64_t)lane * E + e] : 0.0f;
    for (int r0 = 0; r0 < rows; r0 += kWave) {
        s_v[buf][lane] = v;
        const int rn = r0 + kWave + lane;
        v = rn < rows ? weights[(int64_t)rn * E + e] : 0.0f;
        __syncthreads();
        if (lane == 0) {
            const int n = min(kWave, rows - r0);
            for (int i = 0; i < n; ++i) total = total + s_v[buf][i];
        }
        buf ^= 1;
    }
    if (lane == 0) loads[e] = total;
}

}  // namespace nsosx

using namespace nsosx;

extern "C" int64_t nsosx_moe_route_workspace(int rows, int experts) {
    if (rows <= 0 || experts <= 0) return 0;
    const int64_t nblocks = (rows + kRouteBlock - 1) / kRouteBlock;
    return nblocks * experts;
}

extern "C" int nsosx_moe_route(const float* logits, const uint8_t* valid_rows, int rows,
                               int experts, int k, float* weights, int32_t* selected,
                               int32_t* counts, int32_t* offsets, int32_t* perm, int32_t* slot_of,
                               float* loads, int32_t* workspace, void* stream) {
    // counts/offsets/perm/slot_of/workspace all NULL: selection only (the sparse decode
    // reads selected and weights and needs no expert-major permutation)
    const bool select_only = !counts && !offsets && !perm && !slot_of && !workspace;
    if (!logits || !weights || !selected ||
        (!select_only && (!counts || !offsets || !perm || !slot_of || !workspace)))
        return fail(NSOSX_ERR_INVALID, "moe_route: null pointer");
    if (rows <= 0 || experts <= 0 || experts > kMaxExperts || k <= 0 || k > experts)
        return fail(NSOSX_ERR_INVALID, "moe_route: need rows > 0, 0 < k <= E <= 64");
    if ((int64_t)rows * k > 2147483647LL) return fail(NSOSX_ERR_OVERFLOW, "moe_route: rows*k too large");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int nblocks = (rows + kRouteBlock - 1) / kRouteBlock;
    const dim3 rgrid((rows + 255) / 256), rblock(256);
    if (!select_only && (int64_t)nblocks * experts <= kPlaceMaxCounts) {
        // two launches: routing + block counts, then scans + stable ranks
        if (experts <= 8)
            hipLaunchKernelGGL(route_rows_count_kernel<8>, dim3(nblocks), rblock, 0, st, logits,
                               valid_rows, rows, experts, k, weights, selected, workspace);
        else if (experts <= 16)
            hipLaunchKernelGGL(route_rows_count_kernel<16>, dim3(nblocks), rblock, 0, st, logits,
                               valid_rows, rows, experts, k, weights, selected, workspace);
        else
            hipLaunchKernelGGL(route_rows_count_kernel<kMaxExperts>, dim3(nblocks), rblock, 0, st,
                               logits, valid_rows, rows, experts, k, weights, selected, workspace);
        hipLaunchKernelGGL(route_place_kernel, dim3(nblocks), rblock, 0, st, selected, rows,
                           experts, k, nblocks, workspace, counts, offsets, perm, slot_of);
        if (loads)
            hipLaunchKernelGGL(route_loads_kernel, dim3(experts), dim3(kWave), 0, st, weights,
                               rows, experts, loads);
        return check_launch("moe_route");
    }
    if (experts <= 8)
        hipLaunchKernelGGL(route_rows_kernel<8>, rgrid, rblock, 0, st, logits, valid_rows, rows,
                           experts, k, weights, selected);
    else if (experts <= 16)
        hipLaunchKernelGGL(route_rows_kernel<16>, rgrid, rblock, 0, st, logits, valid_rows, rows,
                           experts, k, weights, selected);
    else
        hipLaunchKernelGGL(route_rows_kernel<kMaxExperts>, rgrid, rblock, 0, st, logits,
                           valid_rows, rows, experts, k, weights, selected);
    if (loads)
        hipLaunchKernelGGL(route_loads_kernel, dim3(experts), dim3(kWave), 0, st, weights, rows,
                           experts, loads);
    if (select_only) return check_launch("moe_route");
    hipLaunchKernelGGL(route_count_kernel, dim3(nblocks), dim3(kRouteBlock), 0, st, selected, rows,
                       experts, k, workspace);
    hipLaunchKernelGGL(route_scan_kernel, dim3(1), dim3(64), 0, st, workspace, nblocks, experts,
                       counts, offsets);
    hipLaunchKernelGGL(route_assign_kernel, dim3(nblocks), dim3(kRouteBlock), 0, st, selected, rows,
                       experts, k, workspace, offsets, perm, slot_of);
    return check_launch("moe_route");
}

extern "C" int nsosx_moe_combine(const void* expert_out, int in_dtype, const int32_t* slot_of,
                                 const int32_t* selected, const float* weights, int rows,
                                 int experts, int k, int dim, void* out, int out_dtype,
                                 void* stream) {
    if (!expert_out || !selected || !weights || !out)
        return fail(NSOSX_ERR_INVALID, "moe_combine: null pointer");
    if (rows <= 0 || rows > 65535 * 256 || experts <= 0 || experts > kMaxExperts || k <= 0 ||
        k > experts || dim <= 0)
        return fail(NSOSX_ERR_INVALID, "moe_combine: bad shape");
    if (!valid_dtype(in_dtype) || !valid_dtype(out_dtype))
        return fail(NSOSX_ERR_INVALID, "moe_combine: bad dtype");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const uintptr_t ptrs = reinterpret_cast<uintptr_t>(expert_out) | reinterpret_cast<uintptr_t>(out);
    const uintptr_t align = ptrs & (in_dtype == NSOSX_F32 || out_dtype == NSOSX_F32 ? 15 : 7);
    if (dim % 4 == 0 && align == 0) {
        const dim3 rgrid((rows + 3) / 4), rblock(256);
        const bool v8 = dim % 8 == 0 && (ptrs & 15) == 0;
#define NSOSX_COMBR(I, O)                                                                        \
    if (v8) hipLaunchKernelGGL((combine_rows_kernel<I, O, 8>), rgrid, rblock, 0, st, expert_out, \
                               slot_of, selected, weights, rows, experts, k, dim, out);          \
    else hipLaunchKernelGGL((combine_rows_kernel<I, O, 4>), rgrid, rblock, 0, st, expert_out,    \
                            slot_of, selected, weights, rows, experts, k, dim, out);
        if (in_dtype == NSOSX_F32) {
            if (out_dtype == NSOSX_F32) { NSOSX_COMBR(NSOSX_F32, NSOSX_F32) } else { NSOSX_COMBR(NSOSX_F32, NSOSX_BF16) }
        } else {
            if (out_dtype == NSOSX_F32) { NSOSX_COMBR(NSOSX_BF16, NSOSX_F32) } else { NSOSX_COMBR(NSOSX_BF16, NSOSX_BF16) }
        }
#undef NSOSX_COMBR
        return check_launch("moe_combine");
    }
    if (rows > 65535) return fail(NSOSX_ERR_INVALID, "moe_combine: rows must be <= 65535 when dim % 4 != 0");
    const dim3 grid((dim + 255) / 256, rows), block(256);
#define NSOSX_COMB(I, O)                                                                        \
    hipLaunchKernelGGL((combine_kernel<I, O>), grid, block, 0, st, expert_out, slot_of, selected, \
                       weights, rows, experts, k, dim, out);
    if (in_dtype == NSOSX_F32) {
        if (out_dtype == NSOSX_F32) { NSOSX_COMB(NSOSX_F32, NSOSX_F32) } else { NSOSX_COMB(NSOSX_F32, NSOSX_BF16) }
    } else {
        if (out_dtype == NSOSX_F32) { NSOSX_COMB(NSOSX_BF16, NSOSX_F32) } else { NSOSX_COMB(NSOSX_BF16, NSOSX_BF16) }
    }
#undef NSOSX_COMB
    return check_launch("moe_combine");
}
