// BitLinear decode GEMVs on gfx950: the packed-weight streaming GEMV (M <= 8),
// its grouped forms (decode projections, expert GEMVs) and the sparse MoE decode.
//
// Reference semantics (OXN/nsos/ of vitorGgC569/reimagined):
//   GEMM + affine src/bitnet_adapter_avx2.cpp:52-158
//   packed format src/bitnet_adapter.cpp:570-606
#include "bitlinear.hpp"

namespace nsosx {

// ===========================================================================
// Streaming GEMV (M <= 8).  A row of W is K/16 words; a lane takes a chunk
// of 4 words (64 weights, one 16-byte load) and LPR lanes share a row, LPR
// the smallest power of two >= K/64 (capped at 64), so one wave-load covers
// 64/LPR rows.  The lane's activation chunk is byte-transposed into the
// unpack order once and reused for every row the wave visits; partial sums
// meet in a butterfly over the row's lanes.
// ===========================================================================

// Decode GEMV.  lpr lanes share a row (a lane takes one 64-weight chunk, 16
// bytes), so a wave step covers rpw = 64 / lpr rows.  A wave streams blocks of
// STEPS steps; a lane keeps one partial sum per (step, token row) of the block,
// and the block's sums are combined by a transpose-reduce over the lpr lanes of
// a row (each exchange halves the values a lane holds), so a lane ends with
// complete sums for STEPS / lpr (at least one) of the block's rows.  K > 64*lpr
// (K > 4096) walks a row in several chunk rounds.
constexpr int kGemvDepth = 8;   // weight loads in flight per lane

// row steps per block: fewer for more token rows, so the partial sums stay in registers
template <int MT>
constexpr int gemv_steps() { return MT <= 2 ? 16 : (MT <= 4 ? 8 : 4); }

// A small matrix (fewer than kGemvShortBlocks blocks of the default depth, e.g. a
// 1024 x 2048 projection: 32 waves) is latency-bound: its waves then take
// kGemvShortSteps steps each, all loads of a wave in flight at once, so the matrix is
// spread over several times more waves and a wave waits for one memory round trip
// instead of two.
constexpr int kGemvShortSteps = 4;
constexpr int kGemvShortBlocks = 512;

// lanes that share a row: one 16-byte chunk (64 weights) each, up to the whole wave
__host__ __device__ inline int gemv_lpr(int K) {
    const int cpr = ((K >> 4) + 3) >> 2;
    int lpr = 1;
    while (lpr < cpr && lpr < 64) lpr <<= 1;
    return lpr;
}

// steps per block for `sets` matrices [N, K] in one launch at MT token rows
__host__ __device__ inline int gemv_steps_for(int MT, int N, int K, int sets) {
    const int sd = MT <= 2 ? 16 : (MT <= 4 ? 8 : 4);
    if (sd <= kGemvShortSteps || (K & 63) != 0) return sd;
    const int rows = sd * (64 / gemv_lpr(K));
    const int64_t blocks = (int64_t)((N + rows - 1) / rows) * sets;
    return blocks < kGemvShortBlocks ? kGemvShortSteps : sd;
}

// Weight and activation loads of the GEMV are branch-free, so that the
// compiler counts the loads in flight exactly instead of draining them at every
// branch.  Out-of-range indices are clamped into the buffers instead: a row
// past N is computed but never written, and a chunk or word past the row end
// meets an activation fragment that is zero there.  AL: rows start 16-byte
// aligned (K % 64 == 0), so a chunk is one 16-byte load; otherwise four dword
// loads whose word index is clamped to the matrix.
template <bool AL>
__device__ __forceinline__ uint4 gemv_load_w(const GemvProblem& pb, int n, int c, int W16) {
    n = min(n, pb.N - 1);
    if (AL) {
        c = min(c, (W16 >> 2) - 1);
        return load_stream16(pb.packed + (int64_t)n * W16 + c * 4);
    }
    const int64_t last = (int64_t)pb.N * W16 - 1;
    const int64_t base = (int64_t)n * W16 + (int64_t)c * 4;
    const global_u32* src = (const global_u32*)pb.packed;
    return make_uint4(src[min(base, last)], src[min(base + 1, last)], src[min(base + 2, last)],
                      src[min(base + 3, last)]);
}

// Activation fragment of chunk c (64 values) for token rows 0..MT-1, in the
// order unpack_word() produces; zero where k >= K.  Rows mi >= M read row M-1
// (their sums are never written).
template <int MT>
__device__ __forceinline__ void gemv_load_x(const int8_t* __restrict__ q, int M, int K, int c,
                                            uint32_t xa[MT][4][4]) {
#pragma unroll
    for (int mi = 0; mi < MT; ++mi)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int k = c * 64 + g * 16;
            const int row = min(mi, M - 1);
            const uint4 v = *reinterpret_cast<const uint4*>(q + (int64_t)row * K + min(k, K - 16));
            const uint32_t keep = k < K ? 0xFFFFFFFFu : 0u;
            const uint32_t d[4] = {v.x & keep, v.y & keep, v.z & keep, v.w & keep};
            transpose16(d, xa[mi][g]);
        }
}

template <int MT>
__device__ __forceinline__ void gemv_dot(uint4 w, const uint32_t xa[MT][4][4], int acc[MT]) {
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        uint32_t wv[4];
        unpack_word(ww[g], wv);
#pragma unroll
        for (int mi = 0; mi < MT; ++mi)
#pragma unroll
            for (int s = 0; s < 4; ++s) acc[mi] = sdot4(wv[s], xa[mi][g][s], acc[mi]);
    }
}

// Combines a block's partial sums over the lpr lanes of each row and writes the
// rows.  At offset o, lanes with bit o set keep the upper half of their step
// values and pass the lower half (the halving levels are unrolled, so every
// register index is static); offsets left once a lane holds one value are a
// plain butterfly, and of the lanes holding copies the one with those bits
// clear writes.
template <int MT, int STEPS, int YDT, bool ACC_OUT, bool SQRELU = false>
__device__ __forceinline__ void gemv_finish(int (&part)[STEPS][MT], const GemvProblem& pb,
                                            const float* __restrict__ act_scale, int M, void* y,
                                            int32_t* acc_out, int lr, int lpr, int sub, int rpw,
                                            int n_base) {
    int o = lpr >> 1;
    int cnt = STEPS;
    int sidx = 0;
#pragma unroll
    for (int L = 0; (STEPS >> (L + 1)) > 0; ++L) {
        const int half = STEPS >> (L + 1);
        if (o > 0) {
            const bool hi = (lr & o) != 0;
            // bit-mask select: a ternary here is turned into an indexed register read
            const int hm = hi ? -1 : 0;
#pragma unroll
            for (int s = 0; s < half; ++s)
#pragma unroll
                for (int mi = 0; mi < MT; ++mi) {
                    const int lo_v = part[s][mi], hi_v = part[s + half][mi];
                    const int diff = (lo_v ^ hi_v) & hm;
                    part[s][mi] = (lo_v ^ diff) + __shfl_xor(hi_v ^ diff, o, kWave);
                }
            sidx = (sidx << 1) | (hi ? 1 : 0);
            cnt = half;
            o >>= 1;
        }
    }
    const int low_bits = o > 0 ? (lr & ((o << 1) - 1)) : 0;
    for (; o > 0; o >>= 1)
#pragma unroll
        for (int mi = 0; mi < MT; ++mi) part[0][mi] += __shfl_xor(part[0][mi], o, kWave);
    if (low_bits != 0) return;
    // the lane's values are steps sidx * cnt .. sidx * cnt + cnt - 1 of its sub-row
#pragma unroll
    for (int j = 0; j < STEPS; ++j) {
        if (j < cnt) {
            const int n = n_base + (sidx * cnt + j) * rpw + sub;
            if (n < pb.N) {
#pragma unroll
                for (int mi = 0; mi < MT; ++mi) {
                    if (mi < M) {
                        if (ACC_OUT) acc_out[(int64_t)mi * pb.N + n] = part[j][mi];
                        if (y) {
                            const float comb = __fmul_rn(act_scale[mi], pb.ws);
                            float v = dequant(part[j][mi], comb, pb.mag, pb.bias, n);
                            if (SQRELU) {
                                v = v > 0.0f ? v : 0.0f;
                                v = __fmul_rn(v, v);
                            }
                            store_act<YDT>(y, (int64_t)mi * pb.N + n, v);
                        }
                    }
                }
            }
        }
    }
}

// A wave walks its items (row block, chunk round, step) in order and keeps the
// weight loads of the next D items in flight, across round and block
// boundaries.  The activation fragment stays in registers while K <= 64 * lpr
// (one round); longer rows reload it at each round.
template <int MT, int YDT, bool ACC_OUT, bool AL, int STEPS, bool SQRELU = false>
__device__ __forceinline__ void gemv_body_impl(const GemvProblem& pb,
                                               const int8_t* __restrict__ q,
                                               const float* __restrict__ act_scale, int M,
                                               void* y, int32_t* acc_out, int wave_id,
                                               int num_waves) {
    const int lane = threadIdx.x & 63;
    const int W16 = pb.K >> 4;
    const int cpr = (W16 + 3) >> 2;            // 4-word chunks per row
    int lpr = 1;
    while (lpr < cpr && lpr < 64) lpr <<= 1;   // lanes per row
    const int rpw = 64 / lpr;                  // rows per wave step
    const int lr = lane & (lpr - 1);
    const int sub = lane / lpr;
    const int rounds = (cpr + lpr - 1) / lpr;
    // unaligned rows (rare: K % 64 != 0) keep only two items in flight, as their four
    // word addresses per item would otherwise raise the register count of the kernel
    constexpr int DW = AL ? kGemvDepth : 2;
    constexpr int D = STEPS < DW ? STEPS : DW;
    const int rows_per_block = STEPS * rpw;
    const int nblocks = (pb.N + rows_per_block - 1) / rows_per_block;
    if (wave_id >= nblocks) return;

    uint32_t xa[MT][4][4];
    gemv_load_x<MT>(q, M, pb.K, lr, xa);
    uint4 ring[D];
#pragma unroll
    for (int d = 0; d < D; ++d)
        ring[d] = gemv_load_w<AL>(pb, (wave_id * STEPS + d) * rpw + sub, lr, W16);
    for (int blk = wave_id; blk < nblocks; blk += num_waves) {
        int part[STEPS][MT];
#pragma unroll
        for (int s = 0; s < STEPS; ++s)
#pragma unroll
            for (int mi = 0; mi < MT; ++mi) part[s][mi] = 0;
        for (int r = 0; r < rounds; ++r) {
            if (rounds > 1 && (r > 0 || blk != wave_id)) gemv_load_x<MT>(q, M, pb.K, r * lpr + lr, xa);
            // the item D ahead of step s lies in this round, the next round of this
            // block, or round 0 of the wave's next block
            const bool last_round = r + 1 == rounds;
            const int nb_next = last_round ? blk + num_waves : blk;
            const int c_next = (last_round ? 0 : r + 1) * lpr + lr;
            const int c_cur = r * lpr + lr;
#pragma unroll
            for (int s = 0; s < STEPS; ++s) {
                const uint4 cur = ring[s % D];
                const int s2 = s + D;
                if (s2 < STEPS)
                    ring[s % D] = gemv_load_w<AL>(pb, (blk * STEPS + s2) * rpw + sub, c_cur, W16);
                else
                    ring[s % D] = gemv_load_w<AL>(pb, (nb_next * STEPS + s2 - STEPS) * rpw + sub,
                                                  c_next, W16);
                gemv_dot<MT>(cur, xa, part[s]);
            }
        }
        gemv_finish<MT, STEPS, YDT, ACC_OUT, SQRELU>(part, pb, act_scale, M, y, acc_out, lr, lpr, sub,
                                             rpw, blk * rows_per_block);
    }
}

template <int MT, int YDT, bool ACC_OUT, bool SQRELU = false>
__device__ __forceinline__ void gemv_body_long(const GemvProblem& pb,
                                               const int8_t* __restrict__ q,
                                               const float* __restrict__ act_scale, int M,
                                               void* y, int32_t* acc_out, int wave_id,
                                               int num_waves, int sets) {
    constexpr int SD = gemv_steps<MT>();
    if ((pb.K & 63) != 0)
        gemv_body_impl<MT, YDT, ACC_OUT, false, SD, SQRELU>(pb, q, act_scale, M, y, acc_out,
                                                            wave_id, num_waves);
    else if (SD > kGemvShortSteps && gemv_steps_for(MT, pb.N, pb.K, sets) == kGemvShortSteps)
        gemv_body_impl<MT, YDT, ACC_OUT, true, kGemvShortSteps, SQRELU>(pb, q, act_scale, M, y,
                                                                        acc_out, wave_id,
                                                                        num_waves);
    else
        gemv_body_impl<MT, YDT, ACC_OUT, true, SD, SQRELU>(pb, q, act_scale, M, y, acc_out,
                                                           wave_id, num_waves);
}

template <int MT, int YDT, bool ACC_OUT>
__global__ __launch_bounds__(256) void gemv_kernel(GemvProblem pb, const int8_t* __restrict__ q,
                                                   const float* __restrict__ act_scale, int M,
                                                   void* y, int32_t* acc_out) {
    // wave-uniform (readfirstlane): the tile loops then branch on scalars, with exact
    // memory wait counts
    const int wave_id = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    const int num_waves = gridDim.x * 4;
    gemv_body_long<MT, YDT, ACC_OUT>(pb, q, act_scale, M, y, acc_out, wave_id, num_waves, 1);
}


// Group g multiplies views[view_sel ? view_sel[g] : g] with activation rows
// q + (g / q_div) * q_stride (q_div > 1: consecutive groups share one input,
// e.g. the k experts a decode token is routed to).  skip_skinny: groups that
// grouped_skinny_kernel takes are left to it.
template <int MT, int YDT, bool SQRELU>
__global__ __launch_bounds__(256) void grouped_gemv_kernel(const nsosx_linear_view* views,
                                                           const int32_t* __restrict__ view_sel,
                                                           const int8_t* __restrict__ q,
                                                           int64_t q_stride, int q_div,
                                                           const float* __restrict__ act_scale,
                                                           int64_t scale_stride, int M, void* y,
                                                           int64_t y_stride, int skip_skinny) {
    const int g = blockIdx.y;
    // a selection of -1 (a padding row of the routing) names no view: nothing to do
    const int vi = view_sel ? view_sel[g] : g;
    if (vi < 0) return;
    const nsosx_linear_view v = views[vi];
    char* yb = static_cast<char*>(y) + g * y_stride * (YDT == NSOSX_F32 ? 4 : 2);
    if (skip_skinny && skinny_group(v, yb)) return;
    GemvProblem pb{v.packed, v.magnitude, v.bias, v.weight_scale, v.outputs, v.inputs};
    // wave-uniform (readfirstlane): the tile loops then branch on scalars, with exact
    // memory wait counts
    const int wave_id = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    const int num_waves = gridDim.x * 4;
    const int gi = g / q_div;
    gemv_body_long<MT, YDT, false, SQRELU>(pb, q + gi * q_stride, act_scale + gi * scale_stride,
                                           M, yb, nullptr, wave_id, num_waves, gridDim.y);
}

static int gemv_blocks(int N, int K, int M) {
    const int rows = gemv_steps_for(M, N, K, 1) * (64 / gemv_lpr(K));
    return (N + rows - 1) / rows;
}

static int gemv_grid(int N, int K, int M) {
    // one row block per wave, up to four rounds of 8 resident waves per CU on 256 CUs
    const int waves = std::min(gemv_blocks(N, K, M), 256 * 8 * 4);
    return std::max(1, (waves + 3) / 4);
}

// The faithful Mamba-2 decode step's out_proj for one row with the gated norm and
// its int8 quantization as a prologue: every workgroup forms the row's codes and
// act_scale in LDS (m2_norm_row: the same operations as mamba2_step_norm_kernel,
// so the same bits; workgroup 0 also shifts the B / C ring slots and writes the
// codes and scale out), then its waves run the M = 1 GEMV on them.  One launch
// where the norm kernel and the GEMV were two.
constexpr int kM2GemvMaxK = 4096;

template <int ADT, int YDT>
__global__ __launch_bounds__(256) void mamba2_norm_gemv_kernel(M2StepArgs a, GemvProblem pb,
                                                               void* out) {
    __shared__ __attribute__((aligned(16))) float s_g[kM2GemvMaxK];
    __shared__ __attribute__((aligned(16))) int8_t s_q[kM2GemvMaxK];
    __shared__ float s_red[4];
    __shared__ float s_inv, s_scale;
    m2_norm_row<ADT, 256, kM2GemvMaxK / (256 * 4)>(a, 0, blockIdx.x == 0, s_q, &s_scale, s_g,
                                                   s_red, &s_inv);
    __syncthreads();
    if (blockIdx.x == 0) {
        for (int i = threadIdx.x * 4; i < pb.K; i += 256 * 4)
            *reinterpret_cast<uint32_t*>(a.q + i) = *reinterpret_cast<const uint32_t*>(s_q + i);
        if (threadIdx.x == 0) a.act_scale[0] = s_scale;
    }
    const int wave_id = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    gemv_body_long<1, YDT, false>(pb, s_q, &s_scale, 1, out, nullptr, wave_id, gridDim.x * 4, 1);
}

template <int YDT>
static void launch_gemv_t(const GemvProblem& pb, const int8_t* q, const float* as, int M,
                          void* y, int32_t* acc, hipStream_t st) {
    const dim3 grid(gemv_grid(pb.N, pb.K, M)), block(256);
#define NSOSX_GEMV(MT)                                                                       \
    if (acc)                                                                                 \
        hipLaunchKernelGGL((gemv_kernel<MT, YDT, true>), grid, block, 0, st, pb, q, as, M, y, \
                           acc);                                                             \
    else                                                                                     \
        hipLaunchKernelGGL((gemv_kernel<MT, YDT, false>), grid, block, 0, st, pb, q, as, M, y, \
                           acc);
    if (M == 1) { NSOSX_GEMV(1) }
    else if (M == 2) { NSOSX_GEMV(2) }
    else if (M <= 4) { NSOSX_GEMV(4) }
    else { NSOSX_GEMV(8) }
#undef NSOSX_GEMV
}

// Grouped decode projections of one input row (GpuProjectionGroup::forward,
// src/gpu_projection_group.cpp:12-49): blockIdx.y = view.  A packed view's
// workgroups with row blocks to run quantize the row themselves into LDS
// (quantize_row_wg: nsosx_quantize_act_i8's operations) and run the M = 1 GEMV on
// it; a float view's waves each take output rows with dot_kernel<.., false, 1>'s
// operations (the row's RMS scale, when asked, from the same in-order sum as
// rms_inv_small_kernel).  Views outside the supported shapes write nothing.
template <int IDT, int ODT>
__global__ __launch_bounds__(256) void decode_proj_kernel(const nsosx_decode_view* __restrict__ views,
                                                          const void* __restrict__ input,
                                                          void* __restrict__ output,
                                                          int64_t output_stride) {
    __shared__ __align__(16) float s_row[kQSmallMaxK];
    __shared__ __align__(16) int8_t s_q[kQSmallMaxK];
    __shared__ float s_red[5];
    __shared__ float s_scale, s_inv;
    const nsosx_decode_view v = views[blockIdx.y];
    constexpr int OES = ODT == NSOSX_F32 ? 4 : 2;
    char* out = static_cast<char*>(output) + (int64_t)blockIdx.y * output_stride * OES;
    const int K = v.inputs, N = v.outputs;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wave_id = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + wave);
    const int num_waves = gridDim.x * 4;
    if (v.packed) {
        if (K <= 0 || (K & 63) != 0 || K > kQSmallMaxK || N <= 0 || v.activation_bits < 2 ||
            v.activation_bits > 8)
            return;
        // workgroups without a row block leave before the prologue
        const int rows = gemv_steps_for(1, N, K, 1) * (64 / gemv_lpr(K));
        if ((int)blockIdx.x * 4 >= (N + rows - 1) / rows) return;
        const float qm = v.activation_bits <= 2 ? 1.0f
                                                : static_cast<float>((1 << (v.activation_bits - 1)) - 1);
        if (v.rms_input)
            quantize_row_wg<IDT, true>(input, 0, K, qm, 1e-6f, s_row, s_red, s_q, &s_scale, nullptr);
        else
            quantize_row_wg<IDT, false>(input, 0, K, qm, 1e-6f, s_row, s_red, s_q, &s_scale, nullptr);
        __syncthreads();
        GemvProblem pb{v.packed, v.magnitude, v.bias, v.weight_scale, N, K};
        gemv_body_long<1, ODT, false>(pb, s_q, &s_scale, 1, out, nullptr, wave_id, num_waves, 1);
        return;
    }
    if (!v.weight || K <= 0 || (K & 3) != 0 || N <= 0 || v.activation_bits != 0 ||
        (reinterpret_cast<uintptr_t>(v.weight) & 15) != 0)
        return;
    if ((int)blockIdx.x * 4 >= N) return;
    float inv = 1.0f;
    if (v.rms_input) {
        if (K > kQSmallMaxK) return;
        for (int k = threadIdx.x; k < K; k += 256) {
            const float t = load_act<IDT>(input, k);
            s_row[k] = (k < (K & ~3)) ? __fmul_rn(t, t) : t;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            float sum = 0.0f;
            for (int k = 0; k < (K & ~3); k += 4) {
                const float4 a = *reinterpret_cast<const float4*>(s_row + k);
                sum = __fadd_rn(sum, a.x);
                sum = __fadd_rn(sum, a.y);
                sum = __fadd_rn(sum, a.z);
                sum = __fadd_rn(sum, a.w);
            }
            const float mean = __fdiv_rn(sum, static_cast<float>(K));
            s_inv = __fdiv_rn(1.0f, sqrtf(__fadd_rn(mean, 1e-6f)));
        }
        __syncthreads();
        inv = s_inv;
    }
    auto load4 = [&](const void* base, bool is_x, int64_t off, float r[4]) {
        if (!is_x || IDT == NSOSX_F32) {
            const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + off);
            r[0] = a.x; r[1] = a.y; r[2] = a.z; r[3] = a.w;
        } else {
            const uint2 a = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + off);
            r[0] = __uint_as_float(a.x << 16); r[1] = __uint_as_float(a.x & 0xFFFF0000u);
            r[2] = __uint_as_float(a.y << 16); r[3] = __uint_as_float(a.y & 0xFFFF0000u);
        }
    };
    for (int row = wave_id; row < N; row += num_waves) {
        float acc = 0.0f;
        for (int k0 = 4 * lane; k0 < K; k0 += 1024) {
            float mine[4][4], other[4][4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int k = min(k0 + 256 * u, K - 4);
                load4(v.weight, false, (int64_t)row * K + k, mine[u]);
                load4(input, true, k, other[u]);
                if (v.rms_input) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) other[u][e] = __fmul_rn(other[u][e], inv);
                }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                if (k0 + 256 * u >= K) break;
#pragma unroll
                for (int e = 0; e < 4; ++e) acc = __fmaf_rn(mine[u][e], other[u][e], acc);
            }
        }
        acc = wave_sum(acc);
        if (lane == 0) {
            if (v.magnitude) acc = __fmul_rn(acc, v.magnitude[row]);
            if (v.bias) acc = __fadd_rn(acc, v.bias[row]);
            store_act<ODT>(out, row, acc);
        }
    }
}

bool mamba2_norm_gemv_ok(int rows, int K) {
    return rows == 1 && K % 64 == 0 && K <= kM2GemvMaxK;
}

int launch_mamba2_norm_gemv(const M2StepArgs& a, int act_dtype, const uint32_t* packed,
                            float weight_scale, int N, const float* magnitude, const float* bias,
                            void* out, int out_dtype, hipStream_t st) {
    const int K = a.H * a.P;
    GemvProblem pb{packed, magnitude, bias, weight_scale, N, K};
    const dim3 grid(gemv_grid(N, K, 1)), block(256);
#define NSOSX_M2G(ADT, YDT) \
    hipLaunchKernelGGL((mamba2_norm_gemv_kernel<ADT, YDT>), grid, block, 0, st, a, pb, out);
    if (act_dtype == NSOSX_F32) {
        if (out_dtype == NSOSX_F32) { NSOSX_M2G(NSOSX_F32, NSOSX_F32) } else { NSOSX_M2G(NSOSX_F32, NSOSX_BF16) }
    } else {
        if (out_dtype == NSOSX_F32) { NSOSX_M2G(NSOSX_BF16, NSOSX_F32) } else { NSOSX_M2G(NSOSX_BF16, NSOSX_BF16) }
    }
#undef NSOSX_M2G
    return check_launch("mamba2_step_out");
}

void launch_gemv(const GemvProblem& pb, const int8_t* q, const float* as, int M, void* y,
                 int y_dtype, int32_t* acc, hipStream_t st) {
    if (y_dtype == NSOSX_F32) launch_gemv_t<NSOSX_F32>(pb, q, as, M, y, acc, st);
    else launch_gemv_t<NSOSX_BF16>(pb, q, as, M, y, acc, st);
}

}  // namespace nsosx

using namespace nsosx;

extern "C" int nsosx_grouped_decode_projections(const nsosx_decode_view* views_dev, int groups,
                                                const void* input, int in_dtype, void* output,
                                                int64_t output_stride, int out_dtype,
                                                void* stream) {
    if (!views_dev || !input || !output)
        return fail(NSOSX_ERR_INVALID, "grouped_decode_projections: null pointer");
    if (groups <= 0 || groups > 65535 || output_stride < 0)
        return fail(NSOSX_ERR_INVALID, "grouped_decode_projections: groups in [1, 65535]");
    if (!valid_dtype(in_dtype) || !valid_dtype(out_dtype))
        return fail(NSOSX_ERR_INVALID, "grouped_decode_projections: bad dtype");
    if (reinterpret_cast<uintptr_t>(input) % 16)
        return fail(NSOSX_ERR_INVALID, "grouped_decode_projections: input must be 16-byte aligned");
    hipStream_t st = static_cast<hipStream_t>(stream);
    // as the grouped GEMV at M = 1: about 8192 workgroups in all, each view's waves
    // striding over its row blocks (or rows)
    const dim3 grid(std::max(4, std::min(512, 8192 / groups)), groups), block(256);
#define NSOSX_DP(I, O) \
    hipLaunchKernelGGL((decode_proj_kernel<I, O>), grid, block, 0, st, views_dev, input, output, \
                       output_stride);
    if (in_dtype == NSOSX_F32) {
        if (out_dtype == NSOSX_F32) { NSOSX_DP(NSOSX_F32, NSOSX_F32) } else { NSOSX_DP(NSOSX_F32, NSOSX_BF16) }
    } else {
        if (out_dtype == NSOSX_F32) { NSOSX_DP(NSOSX_BF16, NSOSX_F32) } else { NSOSX_DP(NSOSX_BF16, NSOSX_BF16) }
    }
#undef NSOSX_DP
    return check_launch("grouped_decode_projections");
}

extern "C" int nsosx_grouped_gemv(const nsosx_linear_view* views_dev, int groups, const int8_t* q,
                                  int64_t q_stride, const float* act_scale, int64_t scale_stride,
                                  int M, void* y, int64_t y_stride, int y_dtype, void* stream) {
    if (!views_dev || !q || !act_scale || !y) return fail(NSOSX_ERR_INVALID, "grouped_gemv: null");
    if (groups <= 0 || groups > 65535 || M <= 0 || M > 8)
        return fail(NSOSX_ERR_INVALID, "grouped_gemv: groups in [1, 65535], M in [1, 8]");
    if (!valid_dtype(y_dtype)) return fail(NSOSX_ERR_INVALID, "grouped_gemv: bad dtype");
    hipStream_t st = static_cast<hipStream_t>(stream);
    // view shapes live on the device, so the grid is sized from the group count alone,
    // each wave striding over its view's row blocks: at M = 1 about 8192 workgroups in
    // all (four rounds of the resident limit at 8 waves per SIMD: short waves balance
    // better than long ones), at M >= 2 about 2048 (most groups usually leave this
    // launch to the skinny one)
    const int per_group = std::max(4, std::min(512, (M == 1 ? 8192 : 2048) / groups));
    const dim3 grid(per_group, groups), block(256);
#define NSOSX_GG(MT, SKIP)                                                                    \
    if (y_dtype == NSOSX_F32)                                                                 \
        hipLaunchKernelGGL((grouped_gemv_kernel<MT, NSOSX_F32, false>), grid, block, 0, st,    \
                           views_dev, nullptr, q, q_stride, 1, act_scale, scale_stride, M, y,  \
                           y_stride, SKIP);                                                   \
    else                                                                                      \
        hipLaunchKernelGGL((grouped_gemv_kernel<MT, NSOSX_BF16, false>), grid, block, 0, st,   \
                           views_dev, nullptr, q, q_stride, 1, act_scale, scale_stride, M, y,  \
                           y_stride, SKIP);
    // M >= 2: the skinny MFMA launch takes the groups it accepts (its stores address y
    // with 32-bit offsets), then the VALU GEMV launch the rest
    const int skip = M >= 2 && (int64_t)groups * y_stride * 4 < ((int64_t)1 << 31);
    if (skip) {
        // about 512 workgroups in all (2 per CU at 64 KB of LDS), so each wave
        // streams several tiles past its workgroup's fragment staging
        const dim3 gsk(std::max(2, std::min(512, 512 / groups)), groups);
        launch_grouped_skinny(gsk, views_dev, q, q_stride, act_scale, scale_stride, M, y, y_stride,
                              y_dtype, st);
    }
    if (M == 1) { NSOSX_GG(1, 0) }
    else if (M == 2) { NSOSX_GG(2, skip) }
    else if (M <= 4) { NSOSX_GG(4, skip) }
    else { NSOSX_GG(8, skip) }
#undef NSOSX_GG
    return check_launch("grouped_gemv");
}

// ===========================================================================
// Sparse MoE decode (launch_moe_sparse_decode, src/cuda/moe_kernels.cu:786-795;
// CPU semantics JambaBlock::forward_moe, src/jamba.cpp:3865-3972): for every
// decode row and each of its k routed experts, up BitLinear -> squared ReLU ->
// down BitLinear as grouped GEMVs over (row, expert) pairs, then the weighted
// combine in ascending expert order.  The row is quantized once for all of its
// experts.  Workspace layout (256-byte aligned sections): q1 int8 [rows, dim],
// s1, r1 f32 [rows], h f32 [rows*k, hidden], q2 int8 [rows*k, hidden],
// s2, r2 f32 [rows*k], o f32 [rows*k, dim].
// ===========================================================================
namespace {
struct SparseWs {
    int8_t* q1; float* s1; float* r1; float* h; int8_t* q2; float* s2; float* r2; float* o;
    int64_t bytes;
};
SparseWs sparse_layout(char* base, int rows, int k, int dim, int hidden) {
    int64_t off = 0;
    auto take = [&](int64_t n) {
        const int64_t at = off;
        off += (n + 255) & ~int64_t(255);
        return base ? base + at : nullptr;
    };
    const int64_t slots = (int64_t)rows * k;
    SparseWs w;
    w.q1 = reinterpret_cast<int8_t*>(take((int64_t)rows * dim));
    w.s1 = reinterpret_cast<float*>(take(4LL * rows));
    w.r1 = reinterpret_cast<float*>(take(4LL * rows));
    w.h = reinterpret_cast<float*>(take(4 * slots * hidden));
    w.q2 = reinterpret_cast<int8_t*>(take(slots * hidden));
    w.s2 = reinterpret_cast<float*>(take(4 * slots));
    w.r2 = reinterpret_cast<float*>(take(4 * slots));
    w.o = reinterpret_cast<float*>(take(4 * slots * dim));
    w.bytes = off;
    return w;
}
}  // namespace

extern "C" int64_t nsosx_moe_sparse_decode_workspace(int rows, int k, int dim, int hidden) {
    if (rows <= 0 || k <= 0 || dim <= 0 || hidden <= 0) return -1;
    return sparse_layout(nullptr, rows, k, dim, hidden).bytes;
}

extern "C" int nsosx_moe_sparse_decode(const nsosx_linear_view* up_views,
                                       const nsosx_linear_view* down_views, int experts, int k,
                                       const int32_t* selected, const float* weights,
                                       const void* x, int x_dtype, int rows, int dim, int hidden,
                                       int rms_input, void* workspace, void* out, int out_dtype,
                                       void* stream) {
    if (!up_views || !down_views || !selected || !weights || !x || !workspace || !out)
        return fail(NSOSX_ERR_INVALID, "moe_sparse_decode: null pointer");
    if (rows <= 0 || experts <= 0 || experts > 64 || k <= 0 || k > experts || dim <= 0 || hidden <= 0 ||
        (int64_t)rows * k > 65535)
        return fail(NSOSX_ERR_INVALID, "moe_sparse_decode: bad shape (rows * k <= 65535)");
    if (!valid_dtype(x_dtype) || !valid_dtype(out_dtype))
        return fail(NSOSX_ERR_INVALID, "moe_sparse_decode: bad dtype");
    const SparseWs w = sparse_layout(static_cast<char*>(workspace), rows, k, dim, hidden);
    hipStream_t st = static_cast<hipStream_t>(stream);
    int rc = nsosx_quantize_act_i8(x, x_dtype, rows, dim, 8, rms_input, w.q1, w.s1, w.r1, stream);
    if (rc) return rc;
    const int slots = rows * k;
    const dim3 block(256);
    const dim3 grid_up(std::max(1, std::min(512, 2048 / slots)), slots);
    // up: group g = (row g / k, expert selected[g]); the k groups of a row share its codes
    hipLaunchKernelGGL((grouped_gemv_kernel<1, NSOSX_F32, true>), grid_up, block, 0, st, up_views,
                       selected, w.q1, (int64_t)dim, k, w.s1, (int64_t)1, 1, w.h, (int64_t)hidden,
                       0);
    rc = check_launch("moe_sparse_decode");
    if (rc) return rc;
    rc = nsosx_quantize_act_i8(w.h, NSOSX_F32, slots, hidden, 8, rms_input, w.q2, w.s2, w.r2,
                               stream);
    if (rc) return rc;
    hipLaunchKernelGGL((grouped_gemv_kernel<1, NSOSX_F32, false>), grid_up, block, 0, st,
                       down_views, selected, w.q2, (int64_t)hidden, 1, w.s2, (int64_t)1, 1, w.o,
                       (int64_t)dim, 0);
    rc = check_launch("moe_sparse_decode");
    if (rc) return rc;
    // slot of (row r, choice i) is r * k + i: the combine's identity map
    return nsosx_moe_combine(w.o, NSOSX_F32, nullptr, selected, weights, rows, experts, k, dim,
                             out, out_dtype, stream);
}
