// Mamba selective scan on gfx950: packed ragged prefill (cu_seqlens), the
// decode step, and the depthwise causal convolution that feeds them.
//
// Reference semantics (OXN/nsos/ of vitorGgC569/reimagined):
//   decay terms    src/mamba2.cpp:443-473 (softplus src/mamba2.cpp:718-726)
//   recurrence     src/mamba2.cpp:2602-2675 (faithful CPU scan)
//   decode step    src/mamba2.cpp:4038-4125
//   causal conv    src/mamba2.cpp:1056-1076, bias + SiLU 2437-2446
//   gate           Tensor::silu_gate, src/tensor.cpp:3323-3343 (silu 3261-3282)
//
// decay = exp(-exp(log(delta) + A_log)) of the reference is evaluated as
// exp2(delta * A2) with A2 = -exp(A_log) * log2(e) formed once per (channel,
// state) in double and rounded to float; v_exp_f32 then costs one
// transcendental per (token, channel, state).
#include "common.hpp"
#include "mamba2_step.hpp"

#include <algorithm>
#include <cmath>
#include <string>

namespace nsosx {

__device__ __forceinline__ float softplus_ref(float v) {
    if (v > 20.0f) return v;
    if (v < -20.0f) return expf(v);
    return log1pf(expf(v));
}

__device__ __forceinline__ float a2_from_log(float a_log) {
    return static_cast<float>(-exp(static_cast<double>(a_log)) * 1.4426950408889634);
}

__device__ __forceinline__ float dpp_xor1(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));
}
__device__ __forceinline__ float dpp_xor2(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));
}

// Native-instruction forms of softplus and SiLU for the per-(token, channel)
// terms (v_exp_f32 / v_log_f32 / v_rcp_f32, each about 1 ulp): log1p(e) is
// taken as log(u) * e / (u - 1) with u = 1 + e, which cancels the rounding of
// u (Kahan), so the relative error stays at a few ulp for all dt_raw.
__device__ __forceinline__ float exp_native(float v) {
    return __builtin_amdgcn_exp2f(v * 1.4426950408889634f);
}

__device__ __forceinline__ float softplus_fast(float v) {
    if (v > 20.0f) return v;
    if (v < -20.0f) return expf(v);
    const float e = exp_native(v);
    const float u = 1.0f + e;
    if (u == 1.0f) return e;
    return __builtin_amdgcn_logf(u) * 0.6931471805599453f * (e * __builtin_amdgcn_rcpf(u - 1.0f));
}

__device__ __forceinline__ float silu_fast(float v) {
    return v * __builtin_amdgcn_rcpf(1.0f + exp_native(-v));
}

// ===========================================================================
// Prefill scan.  A workgroup owns 64 channels of one sequence and walks its
// tokens in order; lane l of the workgroup is channel c0 + l/4 and state
// quad q = l%4, holding states n = q*SPL .. q*SPL+SPL-1 in registers.
// Token chunks of TC rows are staged in LDS with the per-(token, channel)
// terms already formed: delta = softplus(dt) and delta*x interleaved (one
// 8-byte read per token), x itself, and B/C of the chunk.  With CONV the
// staged x is the depthwise causal convolution + bias + SiLU of the raw
// input, restarted at the sequence start (each staging thread slides a
// W-tap window down 8 rows of one channel).  After every 4 tokens the four
// lanes of a channel exchange partial readouts with two DPP steps (a 4x4
// transpose-reduce), so each lane finishes one token's sum; the D skip and
// the SiLU(z) gate are applied in the coalesced store pass.
// Requires channels-per-group (H*P/G) to be a multiple of 64 so a workgroup
// sees one B/C group.
// ===========================================================================
constexpr int kScanTC = 32;       // tokens per LDS chunk
constexpr int kScanCh = 64;       // channels per workgroup
constexpr int kMaxConvW = 8;
constexpr int kOrderMax = 64;     // in-kernel longest-first ordering up to this count (more
                                   // sequences: an order pre-pass, nsosx_scan_fwd_planned)

// Workgroup y-index -> sequence, longest sequence first (ties by index), so
// the longest recurrences start first and short ones fill in behind them.
__device__ __forceinline__ int scan_pick_sequence(const int32_t* cu, int num_seqs, int T,
                                                  int32_t* s_order) {
    if (num_seqs > kOrderMax) return blockIdx.y;
    for (int i = threadIdx.x; i < num_seqs; i += blockDim.x) {
        const int a = min(max(cu[i], 0), T);
        const int li = min(max(cu[i + 1], a), T) - a;
        int rank = 0;
        for (int k = 0; k < num_seqs; ++k) {
            const int b = min(max(cu[k], 0), T);
            const int lk = min(max(cu[k + 1], b), T) - b;
            rank += (lk > li) || (lk == li && k < i);
        }
        s_order[rank] = i;
    }
    __syncthreads();
    return s_order[blockIdx.y];
}

// How a launch of the prefill scan kernels maps its work items onto the tokens.  Plain
// launches leave every pointer NULL: item = sequence.  The time-chunked scan
// runs the kernel over chunks of sequences (item = chunk):
//   order      rank -> item (the longest-first order computed once per launch)
//   seq_start  per item: first token of the item's sequence (the causal conv
//              window at a chunk start holds the sequence's previous tokens)
//   init_row   per item: row of init_state to start from (-1: zeros)
//   state_row  per item: row of final_state to write (-1: none)
//   sum_dl     LOCAL pass: per (item, channel) sum of delta over the item
struct QuadPlan {
    const int32_t* order;
    const int32_t* seq_start;
    const int32_t* init_row;
    const int32_t* state_row;
    float* sum_dl;
};

// PH: one A per head (the faithful Mamba-2 block): every state of a channel decays
// alike, one exp per token.  LOCAL: the first pass of the time-chunked scan (the
// recurrence only: each item's end state and sum of delta, no output).  The plan
// fields are read as in scan_quad_kernel.
template <int ADT, int SPL, bool GATE, bool CONV, bool PH = false, bool LOCAL = false>
__global__ __launch_bounds__(256) void scan_fwd_kernel(
    const void* __restrict__ x, int64_t x_stride, const void* __restrict__ dt,
    const float* __restrict__ a_log, int a_per_state, const void* __restrict__ Bm,
    const void* __restrict__ Cm, const float* __restrict__ Dskip, const void* __restrict__ z,
    int64_t z_stride, const int32_t* __restrict__ cu_seqlens, int num_seqs, int total_tokens,
    int H, int P, int N, int G, const float* __restrict__ conv_w, const float* __restrict__ conv_b,
    int W, const float* __restrict__ init_state, float* __restrict__ final_state,
    void* __restrict__ y, QuadPlan plan) {
    constexpr int NPAD = 4 * SPL;
    constexpr int NRAW = CONV ? 8 + kMaxConvW - 1 : 8;
    constexpr int BCPT = (kScanTC * NPAD + 255) / 256;  // B/C elements per thread per chunk
    __shared__ float2 s_dd[kScanTC][kScanCh];
    __shared__ float s_x[kScanTC][kScanCh];
    __shared__ __align__(16) float s_bc[kScanTC][2 * NPAD];
    __shared__ float s_y[kScanTC][kScanCh + 1];
    __shared__ int32_t s_order[kOrderMax];

    const int tid = threadIdx.x;
    const int D = H * P;
    const int GN = G * N;
    const int c0 = blockIdx.x * kScanCh;
    const int seq = plan.order ? plan.order[blockIdx.y]
                               : (plan.seq_start ? (int)blockIdx.y
                                                 : scan_pick_sequence(cu_seqlens, num_seqs,
                                                                      total_tokens, s_order));
    // a malformed cu_seqlens can only shorten a sequence, never address past T
    const int t0 = min(max(cu_seqlens[seq], 0), total_tokens);
    const int t1 = min(max(cu_seqlens[seq + 1], t0), total_tokens);
    const int cl = tid >> 2;          // recurrence: channel within the block
    const int q = tid & 3;            // recurrence: state quad
    const int c = c0 + cl;
    const int h = c / P;
    const int grp = (h * G) / H;
    // staging / store role: channel sc, rows 8*rg .. 8*rg+7 of the chunk
    const int sc = tid & 63;
    const int rg = tid >> 6;
    const int sch = c0 + sc;
    const int sh = sch / P;
    const float sdsk = Dskip[sh];

    float cw[kMaxConvW], cb = 0.0f;
    if (CONV) {
#pragma unroll
        for (int j = 0; j < kMaxConvW; ++j) cw[j] = j < W ? conv_w[(int64_t)sch * W + j] : 0.0f;
        if (conv_b) cb = conv_b[sch];
    }

    float a2[SPL], st[SPL];
    const int irow = plan.init_row ? plan.init_row[seq] : seq;
#pragma unroll
    for (int i = 0; i < SPL; ++i) {
        const int n = q * SPL + i;
        const bool ok = n < N;
        const float al = a_per_state ? a_log[(int64_t)h * N + min(n, N - 1)] : a_log[h];
        a2[i] = ok ? a2_from_log(al) : 0.0f;
        st[i] = (ok && init_state && irow >= 0) ? init_state[((int64_t)irow * D + c) * N + n]
                                                : 0.0f;
    }
    float sdl = 0.0f;  // LOCAL: this lane's channel's sum of delta over the item
    // first token the causal conv window may read: the sequence start (a time chunk that
    // starts inside its sequence takes the sequence's previous raw x)
    const int tw = plan.seq_start ? max(plan.seq_start[seq], 0) : t0;

    // next chunk's global inputs, loaded one chunk ahead of their use
    float raw[NRAW], dtv[8], zv[8], bcv[2][BCPT];
    auto prefetch = [&](int tb) {
        const int tcn = min(kScanTC, t1 - tb);
        const int rbase = 8 * rg;
#pragma unroll
        for (int j = 0; j < NRAW; ++j) {
            const int tr = tb + rbase + j - (CONV ? W - 1 : 0);
            const bool ok = (!CONV || j < 8 + W - 1) && tr >= (CONV ? tw : t0) && tr < tb + tcn;
            raw[j] = ok ? load_act<ADT>(x, (int64_t)tr * x_stride + sch) : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = rbase + i;
            const int64_t t = tb + r;
            dtv[i] = r < tcn ? load_act<ADT>(dt, t * H + sh) : 0.0f;
            zv[i] = (GATE && r < tcn) ? load_act<ADT>(z, t * z_stride + sch) : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < BCPT; ++k) {
            const int e = tid + 256 * k;
            const int r = e / NPAD, n = e % NPAD;
            float bv = 0.0f, cv = 0.0f;
            if (e < kScanTC * NPAD && r < tcn && n < N) {
                const int64_t off = (int64_t)(tb + r) * GN + grp * N + n;
                bv = load_act<ADT>(Bm, off);
                cv = load_act<ADT>(Cm, off);
            }
            bcv[0][k] = bv;
            bcv[1][k] = cv;
        }
    };

    if (t0 < t1) prefetch(t0);
    for (int tb = t0; tb < t1; tb += kScanTC) {
        const int tc = min(kScanTC, t1 - tb);
        // ---- stage the chunk from the prefetched registers ---------------------
        float zcur[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = 8 * rg + i;
            float xv;
            if (CONV) {
                float acc = 0.0f;
#pragma unroll
                for (int j = 0; j < kMaxConvW; ++j)
                    if (j < W) acc = __fmaf_rn(cw[j], raw[i + j], acc);
                xv = r < tc ? silu_fast(acc + cb) : 0.0f;
            } else {
                xv = raw[i];
            }
            const float dl = r < tc ? softplus_fast(dtv[i]) : 0.0f;
            s_dd[r][sc] = make_float2(dl, dl * xv);
            s_x[r][sc] = xv;
            zcur[i] = zv[i];
        }
#pragma unroll
        for (int k = 0; k < BCPT; ++k) {
            const int e = tid + 256 * k;
            if (e < kScanTC * NPAD) {
                const int r = e / NPAD, n = e % NPAD;
                s_bc[r][n] = bcv[0][k];
                s_bc[r][NPAD + n] = bcv[1][k];
            }
        }
        __syncthreads();
        if (tb + kScanTC < t1) prefetch(tb + kScanTC);
        // ---- recurrence, four tokens per transpose-reduce ---------------------
        for (int r0 = 0; r0 < tc; r0 += 4) {
            float part[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int r = r0 + u;  // rows past tc hold delta = 0, B = C = 0: state unchanged
                const float2 dd = s_dd[r][cl];
                float bq[SPL], cq[SPL];
#pragma unroll
                for (int i = 0; i < SPL; ++i) {
                    bq[i] = s_bc[r][q * SPL + i];
                    cq[i] = LOCAL ? 0.0f : s_bc[r][NPAD + q * SPL + i];
                }
                // (PH: padded states carry B = C = 0, so their shared decay is harmless)
                const float aph = PH ? __builtin_amdgcn_exp2f(dd.x * a2[0]) : 0.0f;
                float p = 0.0f;
#pragma unroll
                for (int i = 0; i < SPL; ++i) {
                    const float a = PH ? aph : __builtin_amdgcn_exp2f(dd.x * a2[i]);
                    st[i] = __fmaf_rn(a, st[i], dd.y * bq[i]);
                    if constexpr (!LOCAL) p = __fmaf_rn(st[i], cq[i], p);
                }
                part[u] = p;
                if constexpr (LOCAL) sdl += dd.x;
            }
            if constexpr (LOCAL) continue;
            // lanes q: after xor-2 exchange keep tokens {0,1} (q<2) or {2,3};
            // after xor-1 exchange keep one token: lane q owns token kq.
            const bool hi2 = (q & 2) != 0;
            const float s0 = hi2 ? part[0] : part[2];
            const float s1 = hi2 ? part[1] : part[3];
            const float k0 = hi2 ? part[2] : part[0];
            const float k1 = hi2 ? part[3] : part[1];
            const float m0 = k0 + dpp_xor2(s0);
            const float m1 = k1 + dpp_xor2(s1);
            const bool hi1 = (q & 1) != 0;
            const float send = hi1 ? m0 : m1;
            const float keep = hi1 ? m1 : m0;
            const float tot = keep + dpp_xor1(send);
            const int kq = (hi2 ? 2 : 0) + (hi1 ? 1 : 0);
            s_y[r0 + kq][cl] = tot;
        }
        __syncthreads();
        // ---- D skip, gate, coalesced store of y ---------------------------------
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = 8 * rg + i;
            if (!LOCAL && r < tc) {
                const int64_t t = tb + r;
                float out = __fmaf_rn(sdsk, s_x[r][sc], s_y[r][sc]);
                if (GATE) out = out * silu_fast(zcur[i]);
                store_act<ADT>(y, t * D + sch, out);
            }
        }
        __syncthreads();
    }
    if (LOCAL && q == 0) plan.sum_dl[(int64_t)seq * D + c] = sdl;
    const int frow = plan.state_row ? plan.state_row[seq] : seq;
    if (final_state && frow >= 0) {
#pragma unroll
        for (int i = 0; i < SPL; ++i) {
            const int n = q * SPL + i;
            if (n < N) final_state[((int64_t)frow * D + c) * N + n] = st[i];
        }
    }
}

// ===========================================================================
// Prefill scan, quad form (N <= 16, conv width <= 4).  A workgroup is one
// wave: 16 channels x 4 state quads, each lane holding SPL = N/4 (rounded up)
// states in registers; lane = 4 * channel + quad, or with 16 states (SPL = 4)
// lane = channel + 16 * quad.  The wave walks its sequence in groups of 4
// tokens.  Lane q of a channel forms the per-(token, channel) terms of token
// r0 + q only: the causal convolution (its window read from an 8-slot LDS row
// holding the previous and this group's raw inputs), bias + SiLU, delta =
// softplus(dt) and delta * x; an exchange through the wave's LDS slice then
// hands every lane all four tokens' delta (and delta * x, below 16 states).
// With 16 states the group's delta * x (x) B terms come from one 4-block
// 16 x 16 x 1 f32 MFMA (block k: B of token r0 + k times the lanes' delta * x
// of token r0 + k), whose accumulator layout is the lane layout above: each
// lane receives exactly its 4 states x 4 tokens, the same rounded products as
// 16 multiplies, and the VALU is left the decays, the state updates and the
// readout.  The recurrence runs the four tokens, the 4x4 transpose-reduce
// leaves lane q with the readout of token r0 + q, and lane q applies the D
// skip and the SiLU(z) gate and writes it to the chunk's output rows in LDS; a
// finished 32-token chunk leaves with one 16-byte store per lane.  B and C
// (shared by all channels of a group) are staged per 32-token chunk in the
// wave's own LDS slice, converted to float once.  The
// workgroup is one wave, so its barriers cost no waiting: the raw inputs of a
// group are loaded into registers two groups ahead (two register sets that even
// and odd groups alternate, so no copy waits on a load in flight) and the B/C rows
// of the next chunk one chunk ahead.
// ===========================================================================
typedef float v16f __attribute__((ext_vector_type(16)));
constexpr int kQuadTC = 32;       // tokens per B/C chunk
constexpr int kQuadCh = 16;       // channels per wave
constexpr int kQuadMaxW = 4;
constexpr int kQuadRedStride = 20;  // floats per channel row of the readout transpose
constexpr int kQuadOutStride = 20;  // floats per token row of the staged outputs (16-byte rows)

// Workgroup -> (sequence rank, channel block).  Consecutive workgroup ids go
// round-robin to the 8 XCDs, each with its own L2; this map hands every run of
// 4 channel blocks (4 x 16 channels: one 128-byte line of a bf16 activation
// row) to one XCD, so a line is fetched into one L2 instead of four, while
// the ranks still advance in dispatch order (longest sequences first).
__device__ __forceinline__ void quad_work_item(int& rank, int& cblk) {
    const int nbx = gridDim.x;
    const int total = nbx * gridDim.y;
    const int L = blockIdx.y * nbx + blockIdx.x;
    int lam = L;
    if (L < (total / 32) * 32) lam = (L / 32) * 32 + (L % 8) * 4 + (L / 8) % 4;
    rank = lam / nbx;
    cblk = lam % nbx;
}

// Sequence of the given rank: the rank-th longest (ties by index).
__device__ __forceinline__ int quad_pick_sequence(const int32_t* cu, int num_seqs, int T,
                                                  int target, int* s_pick) {
    if (num_seqs > kOrderMax) return target;
    for (int i = threadIdx.x; i < num_seqs; i += 64) {
        const int a = min(max(cu[i], 0), T);
        const int li = min(max(cu[i + 1], a), T) - a;
        int rank = 0;
        for (int k = 0; k < num_seqs; ++k) {
            const int b = min(max(cu[k], 0), T);
            const int lk = min(max(cu[k + 1], b), T) - b;
            rank += (lk > li) || (lk == li && k < i);
        }
        if (rank == target) *s_pick = i;
    }
    __syncthreads();
    return *s_pick;
}


// softplus_fast() without branches: the three regimes are formed and selected.
__device__ __forceinline__ float softplus_sel(float v) {
    const float e = exp_native(v);
    const float u = 1.0f + e;
    const float mid = __builtin_amdgcn_logf(u) * 0.6931471805599453f * (e * __builtin_amdgcn_rcpf(u - 1.0f));
    return v > 20.0f ? v : (u == 1.0f ? e : mid);
}

// LOCAL: the first pass of the time-chunked scan: the recurrence only (no
// readout, no output), writing each item's end state and sum of delta.
template <int ADT, int SPL, bool GATE, bool CONV, bool PH = false, bool LOCAL = false>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(4))) void scan_quad_kernel(
    const void* __restrict__ x, int64_t x_stride, const void* __restrict__ dt,
    const float* __restrict__ a_log, int a_per_state, const void* __restrict__ Bm,
    const void* __restrict__ Cm, const float* __restrict__ Dskip, const void* __restrict__ z,
    int64_t z_stride, const int32_t* __restrict__ cu_seqlens, int num_seqs, int total_tokens,
    int H, int P, int N, int G, const float* __restrict__ conv_w, const float* __restrict__ conv_b,
    int W, const float* __restrict__ init_state, float* __restrict__ final_state,
    void* __restrict__ y, QuadPlan plan) {
    using raw_t = typename raw_word<ADT>::type;
    constexpr int NP = 4 * SPL;                 // padded states per channel
    constexpr int BCN = NP / 2;                 // states per staging lane (two lanes per row)
    __shared__ __align__(16) float s_bc[2][kQuadTC][NP];
    __shared__ __align__(16) float s_red[kQuadCh * kQuadRedStride];
    __shared__ __align__(16) float2 s_dx[kQuadCh][4];  // {delta, delta * x} of the group's 4 tokens
    __shared__ __align__(16) float s_dl[kQuadCh][4];   // MF: delta of the group's 4 tokens
    __shared__ float s_xw[kQuadCh][8];  // conv window: raw x of the previous and this group
    __shared__ __align__(16) float s_out[kQuadTC][kQuadOutStride];  // the chunk's outputs
    __shared__ int s_pick;

    const int lane = threadIdx.x;
    const int D = H * P;
    const int GN = G * N;
    // MF (16 states): lane = channel + 16 * state quad, the accumulator layout of the
    // 4-block 16 x 16 x 1 f32 MFMA that forms a group's four (delta * x) (x) B products
    constexpr bool MF = SPL == 4;
    const int q = MF ? lane >> 4 : lane & 3;
    const int cl = MF ? lane & 15 : lane >> 2;  // channel of the wave
    // readout transpose slots: channel row of kQuadRedStride floats, state lane j's
    // partial of token k at 4 j + k (row stride padded against bank conflicts)
    const int red_w = cl * kQuadRedStride + 4 * q;
    const int red_r = cl * kQuadRedStride + q;
    int rank, cblk;
    quad_work_item(rank, cblk);
    const int c = cblk * kQuadCh + cl;
    const int h = c / P;
    const int grp = (h * G) / H;
    // uniform across the wave: keeps the token bases in scalar registers
    const int seq = __builtin_amdgcn_readfirstlane(
        plan.order ? plan.order[rank]
                   : (plan.seq_start ? rank
                                     : quad_pick_sequence(cu_seqlens, num_seqs, total_tokens,
                                                          rank, &s_pick)));
    const int t0 = min(max(cu_seqlens[seq], 0), total_tokens);
    const int t1 = min(max(cu_seqlens[seq + 1], t0), total_tokens);
    const int tlast = total_tokens - 1;
    const float dsk = Dskip[h];

    // conv taps right-aligned in kQuadMaxW slots: a width-W filter is the 4-tap
    // filter with leading zero taps, and fma(0, x, 0) leaves the sum at +0
    float cw[kQuadMaxW], cb = 0.0f;
    if (CONV) {
#pragma unroll
        for (int j = 0; j < kQuadMaxW; ++j) {
            const int jw = j - (kQuadMaxW - W);
            cw[j] = jw >= 0 ? conv_w[(int64_t)c * W + jw] : 0.0f;
        }
        if (conv_b) cb = conv_b[c];
    }
    float a2[SPL], st[SPL];
#pragma unroll
    for (int i = 0; i < SPL; ++i) {
        const int n = q * SPL + i;
        const bool ok = n < N;
        const float al = a_per_state ? a_log[(int64_t)h * N + min(n, N - 1)] : a_log[h];
        a2[i] = ok ? a2_from_log(al) : 0.0f;
    }
    {
        const int irow = plan.init_row ? plan.init_row[seq] : seq;
#pragma unroll
        for (int i = 0; i < SPL; ++i) {
            const int n = q * SPL + i;
            st[i] = (n < N && init_state && irow >= 0) ? init_state[((int64_t)irow * D + c) * N + n]
                                                       : 0.0f;
        }
    }
    float sdl = 0.0f;  // LOCAL: running sum of delta

    // Loads are branch-free: indices past the data are clamped to the last row and
    // the values masked where they are used, so the compiler keeps the loads in
    // flight across a whole group (element indices fit in 32 bits; the host checks).
    // B/C staging role: lanes 0-31 stage B, 32-63 stage C; two lanes per chunk row
    // (rows srow and srow + 16), each converting half of the row's states.
    const int sm = lane >> 5;
    const int srow = (lane & 31) >> 1;
    const int shalf = lane & 1;
    const void* smat = sm ? Cm : Bm;
    const bool bc_vec = (SPL == 4) && N == 16 && (GN % 8) == 0 &&
                        ((reinterpret_cast<uintptr_t>(Bm) | reinterpret_cast<uintptr_t>(Cm)) & 15) == 0;
    constexpr int BCW = ADT == NSOSX_F32 ? BCN : (BCN + 1) / 2;  // dwords per lane per row
    // one register set for both load forms, in the vector load's word format (bf16:
    // state 2i in the low half of word i, 2i + 1 in the high half): two arrays chosen
    // by the runtime bc_vec were kept in scratch memory
    uint32_t bcraw[2][BCW];
    int bc_ok = 0;
    auto prefetch_bc = [&](int tb) {
        bc_ok = 0;
#pragma unroll
        for (int pass = 0; pass < 2; ++pass) {
            const int t = tb + srow + 16 * pass;
            bc_ok |= (t < t1 ? 1 : 0) << pass;
            const int base = min(t, tlast) * GN + grp * N + shalf * BCN;
            if (bc_vec) {
                const global_u32x4* src;
                if (ADT == NSOSX_F32) {
                    src = (const global_u32x4*)((const float*)smat + base);
#pragma unroll
                    for (int w4 = 0; w4 < BCW / 4; ++w4) {
                        const u32x4 v = src[w4];
                        bcraw[pass][4 * w4 + 0] = v.x; bcraw[pass][4 * w4 + 1] = v.y;
                        bcraw[pass][4 * w4 + 2] = v.z; bcraw[pass][4 * w4 + 3] = v.w;
                    }
                } else {
                    src = (const global_u32x4*)((const uint16_t*)smat + base);
                    const u32x4 v = src[0];
                    bcraw[pass][0] = v.x; bcraw[pass][1] = v.y;
                    bcraw[pass][2] = v.z; bcraw[pass][3] = v.w;
                }
            } else {
#pragma unroll
                for (int j = 0; j < BCN; ++j) {
                    const int n = shalf * BCN + j;
                    const uint32_t r = n < N ? static_cast<uint32_t>(load_raw<ADT>(smat, base + j)) : 0u;
                    if (ADT == NSOSX_F32) bcraw[pass][j] = r;
                    else if (j & 1) bcraw[pass][j >> 1] |= r << 16;
                    else bcraw[pass][j >> 1] = r;
                }
            }
        }
    };
    auto stage_bc = [&]() {
#pragma unroll
        for (int pass = 0; pass < 2; ++pass) {
            const bool ok = (bc_ok >> pass) & 1;
            float v[BCN];
#pragma unroll
            for (int j = 0; j < BCN; ++j) {
                if (ADT == NSOSX_F32) {
                    v[j] = __uint_as_float(bcraw[pass][j]);
                } else {
                    const uint32_t wd = bcraw[pass][j >> 1];
                    v[j] = __uint_as_float((j & 1) ? (wd & 0xFFFF0000u) : (wd << 16));
                }
            }
#pragma unroll
            for (int j = 0; j < BCN; ++j) s_bc[sm][srow + 16 * pass][shalf * BCN + j] = ok ? v[j] : 0.0f;
        }
    };

    // per-lane token stream through buffer resources: byte offsets of the next group's
    // token (running; past the data the hardware returns 0), raw words two groups ahead
    constexpr uint32_t ES = ADT == NSOSX_F32 ? 4 : 2;
    const uint32_t xs = static_cast<uint32_t>(x_stride) * ES, zs = static_cast<uint32_t>(z_stride) * ES;
    // Each group's resources start at the group's first token (scalar arithmetic:
    // the group base is uniform) and keep the true end of the data as their
    // extent, so the lane offsets stay constant and reads past the end return 0.
    const uint32_t Tn = static_cast<uint32_t>(total_tokens);
    const uint32_t ex = (Tn - 1) * xs + D * ES, edt = Tn * H * ES, ey = Tn * D * ES;
    const uint32_t ez = GATE ? (Tn - 1) * zs + D * ES : 0;
    const uint32_t lx = q * xs + c * ES, ldt = (q * H + h) * ES, lz = q * zs + c * ES;
    const uint32_t ly = (q * D + c) * ES;
    auto group_rsrc = [](const void* base, uint32_t extent, uint32_t off) {
        // extents are below 2^31 (the host checks), so the signed max stays scalar
        const int left = max(static_cast<int>(extent) - static_cast<int>(off), 0);
        return make_rsrc(static_cast<const char*>(base) + off, static_cast<uint32_t>(left));
    };
    uint32_t tnext = static_cast<uint32_t>(t0);  // first token of the group to prefetch
    // set (xr, dtr, zr) feeds the even groups of a chunk, (xr2, dtr2, zr2) the odd ones;
    // a group consumes its set and refills it with the group two ahead (a chunk holds an
    // even number of groups, so the alternation runs on across chunks)
    raw_t xr = 0, dtr = 0, zr = 0, xr2 = 0, dtr2 = 0, zr2 = 0;
    auto load_set = [&](raw_t& xo, raw_t& dto, raw_t& zo) {
        xo = buf_load_raw<ADT>(group_rsrc(x, ex, tnext * xs), lx);
        dto = buf_load_raw<ADT>(group_rsrc(dt, edt, tnext * H * ES), ldt);
        if (GATE) zo = buf_load_raw<ADT>(group_rsrc(z, ez, tnext * zs), lz);
        tnext += 4;
    };

    if (CONV) {
        // the window before t0: zeros at a sequence start; a chunk that starts inside its
        // sequence takes the sequence's previous raw x
        float w0 = 0.0f;
        if (plan.seq_start) {
            const int tt = t0 - 4 + q;
            if (tt >= plan.seq_start[seq] && tt >= 0)
                w0 = load_act<ADT>(x, (int64_t)tt * x_stride + c);
        }
        s_xw[cl][q] = w0;
    }
    // the group whose readout is pending: its conv output, raw gate and base token
    float pv_xv = 0.0f;
    raw_t pv_z = 0;
    int pv_t = t0;
    // Outputs go to the chunk's rows of s_out and leave with one vector store per lane
    // per chunk.  On this architecture a load wait issued while a store is in flight
    // waits for the store as well (loads and stores share one counter and may complete
    // out of order), so a store per group would expose a full store round trip at every
    // group's input wait; per chunk it is one in eight.  Rows of tokens past the sequence
    // hold garbage and are not stored.
    auto finish_readout = [&](float tot) {
        float out = __fmaf_rn(dsk, pv_xv, tot);
        if (GATE) out = out * silu_fast(raw_to_f32<ADT>(pv_z));
        s_out[((pv_t - t0) & (kQuadTC - 1)) + q][cl] = out;
    };
    // lane l stores token row l / 2 of the chunk at tbase, channels 8 (l % 2) .. + 7
    auto flush_out = [&](int tbase) {
        asm volatile("" ::: "memory");
        const int row = lane >> 1, half = lane & 1;
        const float4 v0 = *reinterpret_cast<const float4*>(&s_out[row][half * 8]);
        const float4 v1 = *reinterpret_cast<const float4*>(&s_out[row][half * 8 + 4]);
        asm volatile("" ::: "memory");
        const int tok = tbase + row;
        const uint32_t off = tok < t1
            ? static_cast<uint32_t>(tok * D + cblk * kQuadCh + half * 8) * ES : 0x80000000u;
        const __amdgpu_buffer_rsrc_t ry = make_rsrc(y, ey);
        if constexpr (ADT == NSOSX_F32) {
            __builtin_amdgcn_raw_buffer_store_b128(
                u32x4{__float_as_uint(v0.x), __float_as_uint(v0.y), __float_as_uint(v0.z),
                      __float_as_uint(v0.w)}, ry, off, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b128(
                u32x4{__float_as_uint(v1.x), __float_as_uint(v1.y), __float_as_uint(v1.z),
                      __float_as_uint(v1.w)}, ry, off + 16, 0, 0);
        } else {
            auto pk = [](float lo, float hi) {
                return static_cast<uint32_t>(f32_to_bf16(lo)) |
                       (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
            };
            __builtin_amdgcn_raw_buffer_store_b128(
                u32x4{pk(v0.x, v0.y), pk(v0.z, v0.w), pk(v1.x, v1.y), pk(v1.z, v1.w)}, ry, off,
                0, 0);
        }
    };
    if (t0 < t1) {
        prefetch_bc(t0);
        load_set(xr, dtr, zr);
        load_set(xr2, dtr2, zr2);
    }
    // one 4-token group at chunk row r0 of the chunk at tb, on the given input set
    auto group = [&](const int tb, const int r0, raw_t& xs_, raw_t& dts_, raw_t& zs_) {
            const int tgrp = tb + r0;  // first token of the group (uniform)
            const bool valid = q < t1 - tgrp;
            // B/C of the group's four rows first: the reads overlap the staging math
            // (rows past tc were staged as zero; delta = 0 keeps the state there)
            float bq[4][SPL], cq[4][SPL];
#pragma unroll
            for (int k = 0; k < 4; ++k)
#pragma unroll
                for (int i = 0; i < SPL; ++i) {
                    bq[k][i] = MF ? 0.0f : s_bc[0][r0 + k][q * SPL + i];
                    cq[k][i] = LOCAL ? 0.0f : s_bc[1][r0 + k][q * SPL + i];
                }
            // MF: the MFMA's A operand, B of token r0 + q at state cl
            const float bA = MF ? s_bc[0][r0 + q][cl] : 0.0f;
            // the previous group's readout partials (written at the end of that group)
            float rd0 = 0.0f, rd1 = 0.0f, rd2 = 0.0f, rd3 = 0.0f;
            if constexpr (!LOCAL) {
                rd0 = s_red[red_r]; rd1 = s_red[red_r + 4];
                rd2 = s_red[red_r + 8]; rd3 = s_red[red_r + 12];
            }
            // tokens past the sequence feed only later tokens past it: no mask needed on x
            const float xcur = raw_to_f32<ADT>(xs_);
            const float dtcur = raw_to_f32<ADT>(dts_);
            const raw_t zraw = zs_;
            load_set(xs_, dts_, zs_);
            // ---- per-(token, channel) terms of token tg (formed unconditionally and
            // masked, so the group has no divergent branch) -------------------------
            float xv;
            if (CONV) {
                // the channel's row holds the previous group's raw x in slots 0-3 and
                // this group's in 4-7, so tap j (x[tg - 3 + j]) of token tg = r0 + q is
                // slot q + 1 + j.  LDS operations of one wave complete in order; the
                // compiler barriers keep the other lanes' slots from being read before
                // this group's write or overwritten before the reads.
                float* row = s_xw[cl];
                row[4 + q] = xcur;
                asm volatile("" ::: "memory");
                float acc = 0.0f;
#pragma unroll
                for (int j = 0; j < kQuadMaxW; ++j) acc = __fmaf_rn(row[q + 1 + j], cw[j], acc);
                asm volatile("" ::: "memory");
                row[q] = xcur;  // the next group's previous x
                xv = silu_fast(acc + cb);  // finite; an invalid token's dl = 0 cancels it
            } else {
                xv = xcur;
            }
            const float sp = softplus_sel(dtcur);
            const float dl = valid ? sp : 0.0f;
            const float dx = dl * xv;
            // the quad's four tokens through the wave's LDS slice (LDS operations of one
            // wave complete in order): one or two reads instead of VALU broadcasts
            float dlk[4], dxk[4];
            v16f op = {};
            if constexpr (MF) {
                // block k of the MFMA: B of token r0 + k (A operand, row = state) times
                // delta * x of token r0 + k (B operand, column = channel: lanes 16 k ..
                // 16 k + 15 formed token r0 + k); lane (channel cl, quad q) receives the
                // products for its states 4 q .. 4 q + 3 in registers 4 k .. 4 k + 3.
                // K = 1 and a zero accumulator: each is the rounded product dx * B.
                op = __builtin_amdgcn_mfma_f32_16x16x1f32(bA, dx, v16f{}, 0, 0, 0);
                s_dl[cl][q] = dl;
                const float4 t = *reinterpret_cast<const float4*>(&s_dl[cl][0]);
                dlk[0] = t.x; dlk[1] = t.y; dlk[2] = t.z; dlk[3] = t.w;
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) dxk[kk] = 0.0f;
            } else {
                s_dx[cl][q] = make_float2(dl, dx);
                const float4 t01 = *reinterpret_cast<const float4*>(&s_dx[cl][0]);
                const float4 t23 = *reinterpret_cast<const float4*>(&s_dx[cl][2]);
                dlk[0] = t01.x; dlk[1] = t01.z; dlk[2] = t23.x; dlk[3] = t23.z;
                dxk[0] = t01.y; dxk[1] = t01.w; dxk[2] = t23.y; dxk[3] = t23.w;
            }
            // ---- recurrence over the group's four tokens: all decays first --------
            // (PH, one A per head: every state of the channel decays alike, one exp per
            // token; padded states carry B = C = 0, so their shared decay is harmless)
            float a[4][SPL];
            if constexpr (!PH) {
#pragma unroll
                for (int k = 0; k < 4; ++k)
#pragma unroll
                    for (int i = 0; i < SPL; ++i)
                        a[k][i] = __builtin_amdgcn_exp2f(dlk[k] * a2[i]);
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float ak = __builtin_amdgcn_exp2f(dlk[k] * a2[0]);
#pragma unroll
                    for (int i = 0; i < SPL; ++i) a[k][i] = ak;
                }
            }
            float part[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                float p = 0.0f;
#pragma unroll
                for (int i = 0; i < SPL; ++i) {
                    st[i] = __fmaf_rn(a[k][i], st[i], MF ? op[4 * k + i] : dxk[k] * bq[k][i]);
                    if constexpr (!LOCAL) p = __fmaf_rn(st[i], cq[k][i], p);
                }
                part[k] = p;
            }
            if constexpr (LOCAL) {
                sdl += (dlk[0] + dlk[1]) + (dlk[2] + dlk[3]);
                return;
            }
            // ---- 4x4 transpose through the wave's LDS slice, one group behind:
            // lane q sums token q of the previous group over the channel's four state
            // lanes (its partials were read at the top of this group), then this
            // group's partials are written (LDS operations of one wave complete in
            // order, so the next group's reads see them) -------------------------
            finish_readout(((rd0 + rd1) + rd2) + rd3);
            if (r0 == 0 && tb != t0) flush_out(tb - kQuadTC);  // the previous chunk is complete
            *reinterpret_cast<float4*>(&s_red[red_w]) = make_float4(part[0], part[1], part[2], part[3]);
            pv_xv = xv;
            pv_z = zraw;
            pv_t = tgrp;
    };
    for (int tb = t0; tb < t1; tb += kQuadTC) {
        __syncthreads();  // the previous chunk's B/C reads are done
        stage_bc();
        if (tb + kQuadTC < t1) prefetch_bc(tb + kQuadTC);
        __syncthreads();
        const int tc = min(kQuadTC, t1 - tb);
        for (int r0 = 0; r0 < tc; r0 += 8) {
            group(tb, r0, xr, dtr, zr);
            if (r0 + 4 < tc) group(tb, r0 + 4, xr2, dtr2, zr2);
        }
    }
    if constexpr (!LOCAL) {
        if (t0 < t1) {
            finish_readout(((s_red[red_r] + s_red[red_r + 4]) + s_red[red_r + 8]) +
                           s_red[red_r + 12]);
            flush_out(t0 + ((t1 - 1 - t0) & ~(kQuadTC - 1)));
        }
    } else {
        if (q == 0) plan.sum_dl[(int64_t)seq * D + c] = sdl;
    }
    const int frow = plan.state_row ? plan.state_row[seq] : seq;
    if (final_state && frow >= 0) {
#pragma unroll
        for (int i = 0; i < SPL; ++i) {
            const int n = q * SPL + i;
            if (n < N) final_state[((int64_t)frow * D + c) * N + n] = st[i];
        }
    }
}

// Any shape: one lane per (sequence, channel), states in a loop, in the
// reference's own order of operations.
template <int ADT>
__global__ __launch_bounds__(64) void scan_fwd_generic_kernel(
    const void* __restrict__ x, int64_t x_stride, const void* __restrict__ dt,
    const float* __restrict__ a_log, int a_per_state, const void* __restrict__ Bm,
    const void* __restrict__ Cm, const float* __restrict__ Dskip, const void* __restrict__ z,
    int64_t z_stride, const int32_t* __restrict__ cu_seqlens, int num_seqs, int total_tokens,
    int H, int P, int N, int G, const float* __restrict__ init_state,
    float* __restrict__ final_state, void* __restrict__ y) {
    const int D = H * P;
    const int GN = G * N;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)num_seqs * D) return;
    const int seq = static_cast<int>(idx / D);
    const int c = static_cast<int>(idx % D);
    const int h = c / P;
    const int grp = (h * G) / H;
    float st[64];
    for (int n = 0; n < N; ++n) st[n] = init_state ? init_state[((int64_t)seq * D + c) * N + n] : 0.0f;
    const int t0 = min(max(cu_seqlens[seq], 0), total_tokens);
    const int t1 = min(max(cu_seqlens[seq + 1], t0), total_tokens);
    for (int t = t0; t < t1; ++t) {
        const float xv = load_act<ADT>(x, (int64_t)t * x_stride + c);
        const float dl = softplus_ref(load_act<ADT>(dt, (int64_t)t * H + h));
        float out = Dskip[h] * xv;
        for (int n = 0; n < N; ++n) {
            const float al = a_per_state ? a_log[(int64_t)h * N + n] : a_log[h];
            const float a = __builtin_amdgcn_exp2f(dl * a2_from_log(al));
            const int64_t off = (int64_t)t * GN + grp * N + n;
            st[n] = __fmaf_rn(a, st[n], (dl * load_act<ADT>(Bm, off)) * xv);
            out = __fmaf_rn(st[n], load_act<ADT>(Cm, off), out);
        }
        if (z) out = out * silu_exact(load_act<ADT>(z, (int64_t)t * z_stride + c));
        store_act<ADT>(y, (int64_t)t * D + c, out);
    }
    if (final_state)
        for (int n = 0; n < N; ++n) final_state[((int64_t)seq * D + c) * N + n] = st[n];
}

// ===========================================================================
// Decode step: one token per row against its own state [D, N], in place.
// Lane = (row, channel, state quad); each lane streams its SPL states with
// one 16-byte load and store per 4 states; the four lanes of a channel meet
// with two DPP reductions.
// ===========================================================================
template <int ADT, int SPL, bool GATE>
__global__ __launch_bounds__(256) void scan_step_kernel(
    const void* __restrict__ x, const void* __restrict__ dt, const float* __restrict__ a_log,
    int a_per_state, const void* __restrict__ Bm, const void* __restrict__ Cm,
    const float* __restrict__ Dskip, const void* __restrict__ z, int rows, int H, int P, int N,
    int G, float* __restrict__ state, void* __restrict__ y) {
    const int D = H * P;
    const int GN = G * N;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t lanes = (int64_t)rows * D * 4;
    if (gid >= lanes) return;  // rows * D * 4 is a multiple of 4: whole quads exit together
    const int q = static_cast<int>(gid & 3);
    const int64_t rc = gid >> 2;
    const int r = static_cast<int>(rc / D);
    const int c = static_cast<int>(rc % D);
    const int h = c / P;
    const int grp = (h * G) / H;
    const float xv = load_act<ADT>(x, (int64_t)r * D + c);
    const float dl = softplus_ref(load_act<ADT>(dt, (int64_t)r * H + h));
    const float dx = dl * xv;
    float* sp = state + rc * N + q * SPL;
    float p = 0.0f;
    if (SPL == 4 && N == 16) {
        float4 s4 = *reinterpret_cast<const float4*>(sp);
        float sv[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int n = q * 4 + i;
            const float al = a_per_state ? a_log[(int64_t)h * N + n] : a_log[h];
            const float a = __builtin_amdgcn_exp2f(dl * a2_from_log(al));
            const int64_t off = (int64_t)r * GN + grp * N + n;
            sv[i] = __fmaf_rn(a, sv[i], dx * load_act<ADT>(Bm, off));
            p = __fmaf_rn(sv[i], load_act<ADT>(Cm, off), p);
        }
        *reinterpret_cast<float4*>(sp) = make_float4(sv[0], sv[1], sv[2], sv[3]);
    } else {
#pragma unroll
        for (int i = 0; i < SPL; ++i) {
            const int n = q * SPL + i;
            if (n < N) {
                const float al = a_per_state ? a_log[(int64_t)h * N + n] : a_log[h];
                const float a = __builtin_amdgcn_exp2f(dl * a2_from_log(al));
                const int64_t off = (int64_t)r * GN + grp * N + n;
                const float sv = __fmaf_rn(a, sp[i], dx * load_act<ADT>(Bm, off));
                sp[i] = sv;
                p = __fmaf_rn(sv, load_act<ADT>(Cm, off), p);
            }
        }
    }
    p += dpp_xor2(p);
    p += dpp_xor1(p);
    if (q == 0) {
        float out = __fmaf_rn(Dskip[h], xv, p);
        if (GATE) out = out * silu_exact(load_act<ADT>(z, (int64_t)r * D + c));
        store_act<ADT>(y, (int64_t)r * D + c, out);
    }
}

// ===========================================================================
// Decode step, row-blocked: a workgroup is 64 channels x 4 state quads and
// walks kStepRows rows, so each lane forms its decay exponents A2 (a double exp
// each) once for all those rows.  Per row a lane moves its SPL states with
// vector loads and stores (N = 4 * SPL contiguous floats per channel), the
// per-token terms use the same native softplus / SiLU as the prefill quad
// kernel, and the four lanes of a channel meet with two DPP steps.  The loads of
// all kStepRows rows are issued before the first row is computed.
// ===========================================================================
constexpr int kStepRows = 4;

template <int SPL>
__device__ __forceinline__ void load_states(const float* p, float v[SPL]) {
    if constexpr (SPL == 1) {
        v[0] = p[0];
    } else if constexpr (SPL == 2) {
        const float2 a = *reinterpret_cast<const float2*>(p);
        v[0] = a.x; v[1] = a.y;
    } else {
#pragma unroll
        for (int i = 0; i < SPL; i += 4) {
            const u32x4 a = __builtin_nontemporal_load((global_u32x4*)(p + i));
            v[i] = __uint_as_float(a.x); v[i + 1] = __uint_as_float(a.y);
            v[i + 2] = __uint_as_float(a.z); v[i + 3] = __uint_as_float(a.w);
        }
    }
}

template <int SPL>
__device__ __forceinline__ void store_states(float* p, const float v[SPL]) {
    if constexpr (SPL == 1) {
        p[0] = v[0];
    } else if constexpr (SPL == 2) {
        *reinterpret_cast<float2*>(p) = make_float2(v[0], v[1]);
    } else {
#pragma unroll
        for (int i = 0; i < SPL; i += 4)
            __builtin_nontemporal_store(
                u32x4{__float_as_uint(v[i]), __float_as_uint(v[i + 1]), __float_as_uint(v[i + 2]),
                      __float_as_uint(v[i + 3])},
                (__attribute__((address_space(1))) u32x4*)(p + i));
    }
}

// Lane j's value of the lane's quad, in every lane of the quad (DPP quad_perm(j, j, j, j));
// j must fold to a constant where this is inlined.
template <int J>
__device__ __forceinline__ float quad_bcast_c(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), J * 0x55, 0xF, 0xF, true));
}
__device__ __forceinline__ float quad_bcast(float v, int j) {
    return j == 0 ? quad_bcast_c<0>(v)
                  : j == 1 ? quad_bcast_c<1>(v) : j == 2 ? quad_bcast_c<2>(v) : quad_bcast_c<3>(v);
}

template <int ADT, int SPL, bool GATE, bool VBC>
__global__ __launch_bounds__(256) void scan_step_rows_kernel(
    const void* __restrict__ x, const void* __restrict__ dt, const float* __restrict__ a_log,
    int a_per_state, const void* __restrict__ Bm, const void* __restrict__ Cm,
    const float* __restrict__ Dskip, const void* __restrict__ z, int rows, int H, int P, int N,
    int G, float* __restrict__ state, void* __restrict__ y) {
    const int D = H * P;
    const int GN = G * N;
    const int q = threadIdx.x & 3;
    const int c = blockIdx.x * 64 + (threadIdx.x >> 2);
    if (c >= D) return;  // whole quads leave together
    const int h = c / P;
    const int grp = (h * G) / H;
    const int r0 = blockIdx.y * kStepRows;
    float a2[SPL];
#pragma unroll
    for (int i = 0; i < SPL; ++i) {
        const int n = q * SPL + i;
        a2[i] = a2_from_log(a_per_state ? a_log[(int64_t)h * N + n] : a_log[h]);
    }
    const float dsk = Dskip[h];
    // Rows r0 .. r0 + 3 (kStepRows == the 4 lanes of a channel's quad): lane q forms row
    // r0 + q's per-(row, channel) terms (delta = softplus(dt), delta * x, the gate) once,
    // the quad shares delta and delta * x through DPP broadcasts, and after the readout's
    // transpose-reduce lane q finishes and stores row r0 + q's output.
    static_assert(kStepRows == 4, "one row per lane of a channel's quad");
    float sv[kStepRows][SPL], bq[kStepRows][SPL], cq[kStepRows][SPL];
    const int rq = min(r0 + q, rows - 1);  // rows past the end repeat the last (never stored)
    // VBC (bf16, N = 16, one B / C group per 16 channels: the host checks): the wave's B and
    // C segments of rows r0 .. r0 + 3 (32 bytes each) come in with one 4-byte load per lane
    // (lanes 0-31 B, 32-63 C) and pass through the wave's LDS slice, in place of eight
    // 8-byte loads per wave of the same few lines (13.7 against 14.4 us at config 5)
    __shared__ __align__(16) uint32_t s_bcw[4][64];
    if constexpr (VBC && SPL == 4 && ADT == NSOSX_BF16) {
        const int lane = threadIdx.x & 63;
        const int rr = min(r0 + ((lane & 31) >> 3), rows - 1);
        const uint16_t* m = static_cast<const uint16_t*>(lane < 32 ? Bm : Cm);
        s_bcw[threadIdx.x >> 6][lane] = *reinterpret_cast<const uint32_t*>(
            m + (int64_t)rr * GN + __builtin_amdgcn_readfirstlane(grp) * N + (lane & 7) * 2);
    }
    const float xq = load_act<ADT>(x, (int64_t)rq * D + c);
    const float dtq = load_act<ADT>(dt, (int64_t)rq * H + h);
    const float zq = GATE ? load_act<ADT>(z, (int64_t)rq * D + c) : 0.0f;
#pragma unroll
    for (int j = 0; j < kStepRows; ++j) {
        const int r = min(r0 + j, rows - 1);
        load_states<SPL>(state + ((int64_t)r * D + c) * N + q * SPL, sv[j]);
        const int64_t boff = (int64_t)r * GN + grp * N + q * SPL;
        if constexpr (VBC && SPL == 4 && ADT == NSOSX_BF16) {
            // the quad's four states of row j from the wave's slice (LDS operations of one
            // wave complete in order)
            const uint32_t* sw = s_bcw[threadIdx.x >> 6];
            const uint2 b2 = *reinterpret_cast<const uint2*>(sw + j * 8 + q * 2);
            const uint2 c2 = *reinterpret_cast<const uint2*>(sw + 32 + j * 8 + q * 2);
            bq[j][0] = __uint_as_float(b2.x << 16); bq[j][1] = __uint_as_float(b2.x & 0xFFFF0000u);
            bq[j][2] = __uint_as_float(b2.y << 16); bq[j][3] = __uint_as_float(b2.y & 0xFFFF0000u);
            cq[j][0] = __uint_as_float(c2.x << 16); cq[j][1] = __uint_as_float(c2.x & 0xFFFF0000u);
            cq[j][2] = __uint_as_float(c2.y << 16); cq[j][3] = __uint_as_float(c2.y & 0xFFFF0000u);
        } else {
#pragma unroll
            for (int i = 0; i < SPL; ++i) {
                bq[j][i] = load_act<ADT>(Bm, boff + i);
                cq[j][i] = load_act<ADT>(Cm, boff + i);
            }
        }
    }
    const float dlq = softplus_sel(dtq);
    const float dxq = dlq * xq;
    float part[kStepRows];
#pragma unroll
    for (int j = 0; j < kStepRows; ++j) {
        const float dl = quad_bcast(dlq, j);
        const float dx = quad_bcast(dxq, j);
        float p = 0.0f;
#pragma unroll
        for (int i = 0; i < SPL; ++i) {
            const float a = __builtin_amdgcn_exp2f(dl * a2[i]);
            sv[j][i] = __fmaf_rn(a, sv[j][i], dx * bq[j][i]);
            p = __fmaf_rn(sv[j][i], cq[j][i], p);
        }
        part[j] = p;
        if (r0 + j < rows) store_states<SPL>(state + ((int64_t)(r0 + j) * D + c) * N + q * SPL, sv[j]);
    }
    // transpose-reduce over the quad: lane q ends with row q's sum,
    // (p_q + p_{q^2}) + (p_{q^1} + p_{q^3}) over the lanes' partials
    const bool hi2 = (q & 2) != 0;
    const float s0 = hi2 ? part[0] : part[2];
    const float s1 = hi2 ? part[1] : part[3];
    const float k0 = hi2 ? part[2] : part[0];
    const float k1 = hi2 ? part[3] : part[1];
    const float m0 = k0 + dpp_xor2(s0);
    const float m1 = k1 + dpp_xor2(s1);
    const bool hi1 = (q & 1) != 0;
    const float send = hi1 ? m0 : m1;
    const float keep = hi1 ? m1 : m0;
    const float tot = keep + dpp_xor1(send);
    if (r0 + q < rows) {
        float out = __fmaf_rn(dsk, xq, tot);
        if (GATE) out = out * silu_fast(zq);
        store_act<ADT>(y, (int64_t)(r0 + q) * D + c, out);
    }
}

// ===========================================================================
// Decode step of the faithful Mamba-2 block after its projections, in two
// launches: the conv ring step over x | B | C (mamba2_faithful_conv_step_kernel,
// src/cuda/mamba_kernels.cu:3332-3358), the state step
// (mamba2_faithful_step_kernel, 3376-3404; CPU src/mamba2.cpp:4072-4115), the
// gated norm RMSNorm(y * SiLU(z)) * gamma (4117-4119) and out_proj's int8 input
// quantization (its absmax, act_scale and codes).
//   mamba2_step_scan_kernel, 64 channels of one row per workgroup (the rows'
//     state traffic spread over many CUs): B and C of the workgroup's groups,
//     conv + SiLU into LDS from the ring (read only here), then a quad per x
//     channel as in scan_step_rows_kernel (same operations, same bits): conv +
//     SiLU of x and its ring slots, the states, the readout, y.
//   mamba2_step_norm_kernel, a workgroup per row: the B / C ring slots shifted
//     (after every reader of the previous launch), g = y * SiLU(z), the sum of
//     g^2 by one wave in the element order of the one-wave-per-row gated norm
//     (lane l: elements (c * 64 + l) * 8 + k), inv = 1 / sqrt(mean + eps),
//     normed = g * inv * gamma, the absmax, act_scale and the codes (ties to
//     even over the first inner & ~7 elements, half away from zero after).
// Values are rounded to the activation dtype wherever the unfused chain stores
// them, so the step equals conv_step x3 + selective_scan_step + rmsnorm_gated +
// quantize_act_i8 bit for bit when the gated norm takes its register path
// (inner % 512 == 0, inner <= 4096).
// ===========================================================================
// conv ring value of channel c (conv_step_kernel's order: bias first, taps oldest
// to newest, the new input last) and its SiLU, rounded as stored
template <int ADT>
__device__ __forceinline__ float m2_conv(const M2StepArgs& a, int c, float bias,
                                         const float (&tap)[kM2MaxW - 1], float cur) {
    const int taps = a.W - 1;
    float v = bias;
#pragma unroll
    for (int j = 0; j < kM2MaxW; ++j)
        if (j < a.W) v = __fmaf_rn(a.conv_w[(int64_t)c * a.W + j], j < taps ? tap[j] : cur, v);
    return round_act<ADT>(silu_exact(v));
}

template <int ADT, int SPL>
__global__ __launch_bounds__(256) void mamba2_step_scan_kernel(M2StepArgs a) {
    __shared__ float s_bc[2 * kM2MaxGS];
    const int r = blockIdx.y;
    const int inner = a.H * a.P;
    const int N = a.N, GS = a.G * N;
    const int CD = inner + 2 * GS;
    const int taps = a.W - 1;
    const int q = threadIdx.x & 3;
    const int c0 = blockIdx.x * 64;
    const int c = min(c0 + (threadIdx.x >> 2), inner - 1);  // quads past inner store nothing
    const bool live = c0 + (threadIdx.x >> 2) < inner;
    const int h = c / a.P;
    const int grp = (h * a.G) / a.H;
    // the channel's inputs first: their loads overlap the B / C conv below
    float sv[SPL];
    load_states<SPL>(a.state + ((int64_t)r * inner + c) * N + q * SPL, sv);
    const float* rg = a.ring + (int64_t)r * taps * CD + c;
    float tap[kM2MaxW - 1];
#pragma unroll
    for (int j = 0; j < kM2MaxW - 1; ++j) tap[j] = j < taps ? rg[(int64_t)j * CD] : 0.0f;
    const float cur = load_act<ADT>(a.x, (int64_t)r * inner + c);
    const float bias = a.conv_b ? a.conv_b[c] : 0.0f;
    const float dtv = load_act<ADT>(a.dt, (int64_t)r * a.bcdt_stride + h);
    const float a2 = a2_from_log(a.a_log[h]);
    const float dsk = a.dskip[h];
    // B and C of the groups this workgroup's heads read
    const int g0 = ((c0 / a.P) * a.G) / a.H;
    const int g1 = ((min(c0 + 63, inner - 1) / a.P) * a.G) / a.H;
    const int nv = (g1 - g0 + 1) * N;
    for (int j = threadIdx.x; j < 2 * nv; j += 256) {
        const bool isb = j < nv;
        const int n = g0 * N + (isb ? j : j - nv);           // index within B or C
        const int ch = inner + (isb ? 0 : GS) + n;            // conv channel
        const float bcur = load_act<ADT>(isb ? a.B : a.C, (int64_t)r * a.bcdt_stride + n);
        const float* brg = a.ring + (int64_t)r * taps * CD + ch;
        float btap[kM2MaxW - 1];
#pragma unroll
        for (int t = 0; t < kM2MaxW - 1; ++t) btap[t] = t < taps ? brg[(int64_t)t * CD] : 0.0f;
        s_bc[(isb ? 0 : kM2MaxGS) + j - (isb ? 0 : nv)] =
            m2_conv<ADT>(a, ch, a.conv_b ? a.conv_b[ch] : 0.0f, btap, bcur);
    }
    __syncthreads();
    if (!live) return;  // whole quads leave together
    const float xc = m2_conv<ADT>(a, c, bias, tap, cur);
    if (q == 0) {
        float* wr = a.ring + (int64_t)r * taps * CD + c;
#pragma unroll
        for (int j = 0; j + 1 < kM2MaxW - 1; ++j)
            if (j + 1 < taps) wr[(int64_t)j * CD] = tap[j + 1];
        if (taps > 0) wr[(int64_t)(taps - 1) * CD] = cur;
    }
    // scan_step_rows_kernel's step and readout
    const float dl = softplus_sel(dtv);
    const float dx = dl * xc;
    const float* bq = s_bc + (grp - g0) * N + q * SPL;
    const float* cq = s_bc + kM2MaxGS + (grp - g0) * N + q * SPL;
    float p = 0.0f;
#pragma unroll
    for (int i = 0; i < SPL; ++i) {
        const float dec = __builtin_amdgcn_exp2f(dl * a2);
        sv[i] = __fmaf_rn(dec, sv[i], dx * bq[i]);
        p = __fmaf_rn(sv[i], cq[i], p);
    }
    p += dpp_xor2(p);
    p += dpp_xor1(p);
    store_states<SPL>(a.state + ((int64_t)r * inner + c) * N + q * SPL, sv);
    if (q == 0) store_act<ADT>(a.y, (int64_t)r * inner + c, __fmaf_rn(dsk, xc, p));
}

template <int ADT>
__global__ __launch_bounds__(kM2NormThreads) void mamba2_step_norm_kernel(M2StepArgs a) {
    __shared__ __attribute__((aligned(16))) float s_g[kM2MaxInner];
    __shared__ float s_red[kM2NormThreads / kWave];
    __shared__ float s_inv;
    m2_norm_row<ADT, kM2NormThreads, kM2MaxInner / (kM2NormThreads * 4)>(
        a, blockIdx.x, true, a.q + (int64_t)blockIdx.x * a.H * a.P, a.act_scale + blockIdx.x, s_g,
        s_red, &s_inv);
}

// ===========================================================================
// Depthwise causal convolution + bias + SiLU, restarted per sequence.
// Thread = (token, channel); the sequence start comes from a binary search
// of cu_seqlens.
// ===========================================================================
template <int IDT, int ODT>
__global__ __launch_bounds__(256) void conv1d_kernel(const void* __restrict__ in, int64_t in_stride,
                                                     const float* __restrict__ w,
                                                     const float* __restrict__ bias,
                                                     const int32_t* __restrict__ cu_seqlens,
                                                     int num_seqs, int T, int C, int W, int silu,
                                                     void* __restrict__ out) {
    // thread = (token, channel) over the flat [T, C] output, so few channels (B and C
    // of a group: 16) still fill whole waves
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)T * C) return;
    const int t = static_cast<int>(i / C);
    const int c = static_cast<int>(i - (int64_t)t * C);
    int lo = 0, hi = num_seqs;  // find s with cu[s] <= t < cu[s+1]
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (cu_seqlens[mid] <= t) lo = mid; else hi = mid;
    }
    const int ts = min(max(cu_seqlens[lo], 0), t);  // never reads before token 0
    float acc = 0.0f;
    for (int j = 0; j < W; ++j) {
        const int src = t - (W - 1) + j;
        if (src < ts) continue;
        acc = __fmaf_rn(w[(int64_t)c * W + j], load_act<IDT>(in, (int64_t)src * in_stride + c), acc);
    }
    if (bias) acc = acc + bias[c];
    if (silu) acc = silu_exact(acc);
    store_act<ODT>(out, (int64_t)t * C + c, acc);
}

}  // namespace nsosx

using namespace nsosx;

static int scan_fwd_launch(const void* x, int64_t x_stride, const void* dt, const float* A_log,
                           int a_per_state, const void* B, const void* C, const float* D,
                           const void* z, int64_t z_stride, const int32_t* cu_seqlens,
                           int num_seqs, int total_tokens, int H, int P, int N, int G,
                           int act_dtype, const float* conv_w, const float* conv_b, int conv_width,
                           const float* initial_state, float* final_state, void* y,
                           void* stream, const QuadPlan& plan = QuadPlan{},
                           bool local = false) {
    if (!x || !dt || !A_log || !B || !C || !D || !cu_seqlens || (!y && !local))
        return fail(NSOSX_ERR_INVALID, "selective_scan_fwd: null pointer");
    if (num_seqs <= 0 || num_seqs > 65535 || total_tokens < 0 || H <= 0 || P <= 0 || N <= 0 ||
        N > 64 || G <= 0 || H % G != 0)
        return fail(NSOSX_ERR_INVALID, "selective_scan_fwd: bad shape (N <= 64, H % G == 0)");
    if (!valid_dtype(act_dtype)) return fail(NSOSX_ERR_INVALID, "selective_scan_fwd: bad dtype");
    const int Dm = H * P;
    if (x_stride < Dm || (z && z_stride < Dm))
        return fail(NSOSX_ERR_INVALID, "selective_scan_fwd: row stride smaller than H*P");
    const int per_group = Dm / G;
    const bool conv = conv_w != nullptr;
    if (conv && (conv_width <= 0 || conv_width > kMaxConvW))
        return fail(NSOSX_ERR_INVALID, "conv_scan_fwd: conv width must be in [1, 8]");
    if (conv && !(per_group % kScanCh == 0 ||
                  (N <= 16 && per_group % kQuadCh == 0 && conv_width <= kQuadMaxW)))
        return fail(NSOSX_ERR_INVALID,
                    "conv_scan_fwd: channels per group must be a multiple of 64 (or of 16 with "
                    "N <= 16 and conv width <= 4)");
    hipStream_t st = static_cast<hipStream_t>(stream);
    // the quad kernel addresses rows with 32-bit byte offsets (buffer resources)
    const int64_t max_row = std::max<int64_t>(std::max<int64_t>(x_stride, z ? z_stride : 0),
                                              std::max<int64_t>(Dm, (int64_t)G * N));
    const int64_t esz = act_dtype == NSOSX_F32 ? 4 : 2;
    const bool idx32 = (int64_t)(total_tokens + 8) * max_row * esz < ((int64_t)1 << 31);
    if (N <= 16 && per_group % kQuadCh == 0 && (!conv || conv_width <= kQuadMaxW) && idx32) {
        const dim3 grid(Dm / kQuadCh, num_seqs), block(64);
        const int spl = N <= 4 ? 1 : N <= 8 ? 2 : 4;
        // one A per head with N = 16 (the faithful Mamba-2 block): one decay exp per token
        const bool ph = !a_per_state && spl == 4;
#define NSOSX_QK(ADT, SPL, GATE, CONV, PH, LOC)                                                  \
    hipLaunchKernelGGL((scan_quad_kernel<ADT, SPL, GATE, CONV, PH, LOC>), grid, block, 0, st, x,   \
                       x_stride, dt, A_log, a_per_state, B, C, D, z, z_stride, cu_seqlens,         \
                       num_seqs, total_tokens, H, P, N, G, conv_w, conv_b, conv_width,             \
                       initial_state, final_state, y, plan);
#define NSOSX_QSCAN(ADT, SPL, GATE, CONV)                                                          \
    if (local) {                                                                                   \
        if (SPL == 4 && ph) { NSOSX_QK(ADT, SPL, false, CONV, SPL == 4, true) }                    \
        else { NSOSX_QK(ADT, SPL, false, CONV, false, true) }                                      \
    } else if (SPL == 4 && ph) {                                                                   \
        NSOSX_QK(ADT, SPL, GATE, CONV, SPL == 4, false)                                            \
    } else {                                                                                       \
        NSOSX_QK(ADT, SPL, GATE, CONV, false, false)                                               \
    }
#define NSOSX_QSCAN_C(ADT, SPL, GATE) \
    if (conv) { NSOSX_QSCAN(ADT, SPL, GATE, true) } else { NSOSX_QSCAN(ADT, SPL, GATE, false) }
#define NSOSX_QSCAN_G(ADT, SPL) \
    if (z && !local) { NSOSX_QSCAN_C(ADT, SPL, true) } else { NSOSX_QSCAN_C(ADT, SPL, false) }
#define NSOSX_QSCAN_S(ADT)                          \
    switch (spl) {                                  \
        case 1: NSOSX_QSCAN_G(ADT, 1) break;        \
        case 2: NSOSX_QSCAN_G(ADT, 2) break;        \
        default: NSOSX_QSCAN_G(ADT, 4) break;       \
    }
        if (act_dtype == NSOSX_F32) { NSOSX_QSCAN_S(NSOSX_F32) } else { NSOSX_QSCAN_S(NSOSX_BF16) }
#undef NSOSX_QSCAN_S
#undef NSOSX_QSCAN_G
#undef NSOSX_QSCAN_C
#undef NSOSX_QSCAN
#undef NSOSX_QK
    } else if (per_group % kScanCh == 0) {
        // the LDS-staged form: any N <= 64, conv width <= 8, sequential or time-chunked
        const dim3 grid(Dm / kScanCh, num_seqs), block(256);
        const int spl = N <= 4 ? 1 : N <= 8 ? 2 : N <= 16 ? 4 : N <= 32 ? 8 : 16;
        // one A per head above N = 16 (the faithful Mamba-2 block at the reference's
        // d_state 64): one decay exp per token
        const bool ph = !a_per_state && spl >= 8;
#define NSOSX_SK(ADT, SPL, GATE, CONV, PH, LOC)                                                 \
    hipLaunchKernelGGL((scan_fwd_kernel<ADT, SPL, GATE, CONV, PH, LOC>), grid, block, 0, st, x,   \
                       x_stride, dt, A_log, a_per_state, B, C, D, z, z_stride, cu_seqlens,        \
                       num_seqs, total_tokens, H, P, N, G, conv_w, conv_b, conv_width,            \
                       initial_state, final_state, y, plan);
#define NSOSX_SCAN(ADT, SPL, GATE, CONV)                                                        \
    if (local) {                                                                                \
        if (SPL >= 8 && ph) { NSOSX_SK(ADT, SPL, false, CONV, SPL >= 8, true) }                 \
        else { NSOSX_SK(ADT, SPL, false, CONV, false, true) }                                   \
    } else if (SPL >= 8 && ph) {                                                                \
        NSOSX_SK(ADT, SPL, GATE, CONV, SPL >= 8, false)                                         \
    } else {                                                                                    \
        NSOSX_SK(ADT, SPL, GATE, CONV, false, false)                                            \
    }
#define NSOSX_SCAN_C(ADT, SPL, GATE) \
    if (conv) { NSOSX_SCAN(ADT, SPL, GATE, true) } else { NSOSX_SCAN(ADT, SPL, GATE, false) }
#define NSOSX_SCAN_G(ADT, SPL) \
    if (z && !local) { NSOSX_SCAN_C(ADT, SPL, true) } else { NSOSX_SCAN_C(ADT, SPL, false) }
#define NSOSX_SCAN_S(ADT)                          \
    switch (spl) {                                 \
        case 1: NSOSX_SCAN_G(ADT, 1) break;        \
        case 2: NSOSX_SCAN_G(ADT, 2) break;        \
        case 4: NSOSX_SCAN_G(ADT, 4) break;        \
        case 8: NSOSX_SCAN_G(ADT, 8) break;        \
        default: NSOSX_SCAN_G(ADT, 16) break;      \
    }
        if (act_dtype == NSOSX_F32) { NSOSX_SCAN_S(NSOSX_F32) } else { NSOSX_SCAN_S(NSOSX_BF16) }
#undef NSOSX_SCAN_S
#undef NSOSX_SCAN_G
#undef NSOSX_SCAN_C
#undef NSOSX_SCAN
#undef NSOSX_SK
    } else if (local || plan.seq_start) {
        return fail(NSOSX_ERR_INVALID, "selective_scan_fwd: the time-chunked scan needs channels "
                                       "per group a multiple of 64 (or of 16 with N <= 16 and "
                                       "conv width <= 4)");
    } else {
        const int64_t lanes = (int64_t)num_seqs * Dm;
        const dim3 grid((unsigned)((lanes + 63) / 64)), block(64);
        if (act_dtype == NSOSX_F32)
            hipLaunchKernelGGL(scan_fwd_generic_kernel<NSOSX_F32>, grid, block, 0, st, x, x_stride,
                               dt, A_log, a_per_state, B, C, D, z, z_stride, cu_seqlens, num_seqs,
                               total_tokens, H, P, N, G, initial_state, final_state, y);
        else
            hipLaunchKernelGGL(scan_fwd_generic_kernel<NSOSX_BF16>, grid, block, 0, st, x,
                               x_stride, dt, A_log, a_per_state, B, C, D, z, z_stride, cu_seqlens,
                               num_seqs, total_tokens, H, P, N, G, initial_state, final_state, y);
    }
    return check_launch("selective_scan_fwd");
}

extern "C" int nsosx_selective_scan_fwd(const void* x, int64_t x_stride, const void* dt,
                                        const float* A_log, int a_per_state, const void* B,
                                        const void* C, const float* D, const void* z,
                                        int64_t z_stride, const int32_t* cu_seqlens, int num_seqs,
                                        int total_tokens, int H, int P, int N, int G,
                                        int act_dtype, const float* initial_state,
                                        float* final_state, void* y, void* stream) {
    return scan_fwd_launch(x, x_stride, dt, A_log, a_per_state, B, C, D, z, z_stride, cu_seqlens,
                           num_seqs, total_tokens, H, P, N, G, act_dtype, nullptr, nullptr, 0,
                           initial_state, final_state, y, stream);
}

extern "C" int nsosx_conv_scan_fwd(const void* x_raw, int64_t x_stride, const float* conv_w,
                                   const float* conv_b, int conv_width, const void* dt,
                                   const float* A_log, int a_per_state, const void* B,
                                   const void* C, const float* D, const void* z, int64_t z_stride,
                                   const int32_t* cu_seqlens, int num_seqs, int total_tokens,
                                   int H, int P, int N, int G, int act_dtype,
                                   const float* initial_state, float* final_state, void* y,
                                   void* stream) {
    if (!conv_w) return fail(NSOSX_ERR_INVALID, "conv_scan_fwd: null conv weight");
    return scan_fwd_launch(x_raw, x_stride, dt, A_log, a_per_state, B, C, D, z, z_stride,
                           cu_seqlens, num_seqs, total_tokens, H, P, N, G, act_dtype, conv_w,
                           conv_b, conv_width, initial_state, final_state, y, stream);
}

// ===========================================================================
// Planned scan: a longest-first order computed once per launch (instead of in
// every workgroup), and the time-chunked scan for batches too small to fill
// the GPU (one long prefill).  The chunked scan runs in three launches:
//   1. LOCAL pass over chunks: each chunk's recurrence from zero (the first
//      chunk of a sequence from its initial state), writing the chunk's end
//      state and the sum of delta over it;
//   2. combine, one thread per (sequence, channel, state), sequential over the
//      sequence's chunks: carry[j] = the state entering chunk j, and
//      carry[j+1] = exp2(a2 * sum_delta[j]) * carry[j] + local[j]  (the product
//      of a chunk's decays is exp of the summed exponents);
//   3. the full scan over chunks from carry[j], with the causal conv window of a
//      chunk start taken from the sequence's previous tokens, writing y and,
//      from each sequence's last chunk, its final state.
// ===========================================================================
namespace nsosx {

// Above this many sequences the launch keeps dispatch order: with thousands of short
// sequences every SIMD holds many waves, the tail is short, and ranking them costs more
// than it saves (measured: 1024 sequences of 32-64 tokens ran 13 % slower ranked).
constexpr int kOrderPrepassMax = 512;

__global__ __launch_bounds__(256) void scan_order_kernel(const int32_t* __restrict__ cu, int S,
                                                         int T, int32_t* __restrict__ order) {
    __shared__ int s_len[256];
    const int i = blockIdx.x * 256 + threadIdx.x;
    int li = -1;
    if (i < S) {
        const int a = min(max(cu[i], 0), T);
        li = min(max(cu[i + 1], a), T) - a;
    }
    if (S > kOrderPrepassMax) {
        if (i < S) order[i] = i;
        return;
    }
    int rank = 0;
    for (int base = 0; base < S; base += 256) {
        const int k = base + threadIdx.x;
        int lk = -1;
        if (k < S) {
            const int b = min(max(cu[k], 0), T);
            lk = min(max(cu[k + 1], b), T) - b;
        }
        __syncthreads();
        s_len[threadIdx.x] = lk;
        __syncthreads();
        const int cnt = min(256, S - base);
        for (int j = 0; j < cnt; ++j) {
            const int l = s_len[j];
            rank += (l > li) || (l == li && base + j < i);
        }
    }
    if (i < S) order[rank] = i;
}

// One workgroup: sequence s splits into max(1, ceil(len / C)) chunks, numbered
// in sequence order (an exclusive scan of the counts).
__global__ __launch_bounds__(1024) void chunk_plan_kernel(const int32_t* __restrict__ cu, int S,
                                                          int T, int C, int maxc,
                                                          int32_t* __restrict__ chunk_cu,
                                                          int32_t* __restrict__ seq_start,
                                                          int32_t* __restrict__ init_row,
                                                          int32_t* __restrict__ state_row,
                                                          int32_t* __restrict__ first_chunk) {
    __shared__ int s_scan[1024];
    __shared__ int s_end;
    const int t = threadIdx.x;
    int carry = 0;
    if (t == 0) s_end = 0;
    for (int base = 0; base < S; base += 1024) {
        const int s = base + t;
        int a = 0, l = 0, cnt = 0;
        if (s < S) {
            a = min(max(cu[s], 0), T);
            l = min(max(cu[s + 1], a), T) - a;
            cnt = max(1, (l + C - 1) / C);
        }
        __syncthreads();
        s_scan[t] = cnt;
        __syncthreads();
        for (int off = 1; off < 1024; off <<= 1) {
            const int v = t >= off ? s_scan[t - off] : 0;
            __syncthreads();
            s_scan[t] += v;
            __syncthreads();
        }
        if (s < S) {
            const int first = carry + s_scan[t] - cnt;
            first_chunk[s] = min(first, maxc);  // a malformed cu_seqlens cannot overrun
            for (int j = 0; j < cnt; ++j) {
                const int idx = first + j;
                if (idx >= maxc) break;   // cannot happen: maxc >= S + T / C
                chunk_cu[idx] = a + min(j * C, l);
                seq_start[idx] = a;
                init_row[idx] = j == 0 ? s : -1;
                state_row[idx] = j == cnt - 1 ? s : -1;
            }
            if (s == S - 1) s_end = a + l;
        }
        carry += s_scan[1023];
        __syncthreads();
    }
    __syncthreads();
    for (int idx = min(carry, maxc) + t; idx <= maxc; idx += 1024) {
        chunk_cu[idx] = s_end;
        if (idx < maxc) {
            seq_start[idx] = s_end;
            init_row[idx] = -1;
            state_row[idx] = -1;
        }
    }
    if (t == 0) first_chunk[S] = min(carry, maxc);
}

__global__ __launch_bounds__(256) void chunk_combine_kernel(
    const int32_t* __restrict__ first_chunk, int S, int D, int P, int N,
    const float* __restrict__ a_log, int a_per_state, const float* __restrict__ local,
    const float* __restrict__ sum_dl, const float* __restrict__ init_state,
    float* __restrict__ carry) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)S * D * N) return;
    const int n = static_cast<int>(idx % N);
    const int c = static_cast<int>((idx / N) % D);
    const int s = static_cast<int>(idx / ((int64_t)N * D));
    const int h = c / P;
    const float a2 = a2_from_log(a_per_state ? a_log[(int64_t)h * N + n] : a_log[h]);
    const int j0 = first_chunk[s], j1 = max(first_chunk[s + 1], j0);
    float hs = init_state ? init_state[((int64_t)s * D + c) * N + n] : 0.0f;
    for (int j = j0; j < j1; ++j) {
        const int64_t o = ((int64_t)j * D + c) * N + n;
        carry[o] = hs;
        const float lj = local[o];
        hs = j == j0 ? lj
                     : __fmaf_rn(__builtin_amdgcn_exp2f(a2 * sum_dl[(int64_t)j * D + c]), hs, lj);
    }
}

static int64_t align256(int64_t v) { return (v + 255) & ~int64_t(255); }

// chunk_tokens < 0: chunk when sequences x 16-channel blocks give fewer than two
// waves per SIMD and the sequences are long enough to split; target ~8 waves.
static int resolve_chunk(int S, int T, int H, int P, int N, int chunk_tokens) {
    if (chunk_tokens >= 0) return chunk_tokens;
    const int D = H * P;
    if (S <= 0 || T <= 0 || D % kQuadCh != 0 || (N > 16 && D % kScanCh != 0)) return 0;
    // waves per sequence: 16 channels per wave in either form (the quad kernel's one-wave
    // workgroups, the LDS-staged form's four-wave workgroups of 64 channels)
    const int64_t blocks = D / kQuadCh;
    if ((int64_t)S * blocks >= 2048) return 0;
    int64_t c = ((int64_t)T * blocks + 8191) / 8192;
    c = std::max<int64_t>(c, 64);
    c = std::max<int64_t>(c, ((int64_t)T + 65535 - S - 1) / (65535 - S));  // chunks fit a grid
    c = (c + 31) / 32 * 32;
    if (2 * c > (int64_t)T / S) return 0;
    return static_cast<int>(std::min<int64_t>(c, 1 << 20));
}

struct ScanWs {
    int32_t* order;
    int32_t *chunk_cu, *seq_start, *init_row, *state_row, *first_chunk;
    float *local, *sum_dl, *carry;
    int maxc;
    int64_t bytes;
};

static ScanWs scan_ws_layout(void* base, int S, int T, int D, int N, int C) {
    ScanWs w{};
    int64_t off = 0;
    auto take = [&](int64_t bytes) {
        char* p = base ? static_cast<char*>(base) + off : nullptr;
        off += align256(bytes);
        return p;
    };
    w.order = reinterpret_cast<int32_t*>(take((int64_t)S * 4));
    if (C > 0) {
        const int64_t maxc = (int64_t)S + (T + C - 1) / C;
        w.maxc = static_cast<int>(maxc);
        w.chunk_cu = reinterpret_cast<int32_t*>(take((maxc + 1) * 4));
        w.seq_start = reinterpret_cast<int32_t*>(take(maxc * 4));
        w.init_row = reinterpret_cast<int32_t*>(take(maxc * 4));
        w.state_row = reinterpret_cast<int32_t*>(take(maxc * 4));
        w.first_chunk = reinterpret_cast<int32_t*>(take(((int64_t)S + 1) * 4));
        w.local = reinterpret_cast<float*>(take(maxc * D * N * 4));
        w.sum_dl = reinterpret_cast<float*>(take(maxc * D * 4));
        w.carry = reinterpret_cast<float*>(take(maxc * D * N * 4));
    }
    w.bytes = off;
    return w;
}

}  // namespace nsosx

using namespace nsosx;

extern "C" int64_t nsosx_scan_fwd_workspace(int num_seqs, int total_tokens, int H, int P, int N,
                                            int chunk_tokens) {
    if (num_seqs <= 0 || total_tokens < 0 || H <= 0 || P <= 0 || N <= 0) return 0;
    const int C = resolve_chunk(num_seqs, total_tokens, H, P, N, chunk_tokens);
    return scan_ws_layout(nullptr, num_seqs, total_tokens, H * P, N, C).bytes;
}

extern "C" int nsosx_scan_fwd_planned(const void* x, int64_t x_stride, const float* conv_w,
                                      const float* conv_b, int conv_width, const void* dt,
                                      const float* A_log, int a_per_state, const void* B,
                                      const void* C, const float* D, const void* z,
                                      int64_t z_stride, const int32_t* cu_seqlens, int num_seqs,
                                      int total_tokens, int H, int P, int N, int G, int act_dtype,
                                      const float* initial_state, float* final_state, void* y,
                                      int chunk_tokens, void* workspace, void* stream) {
    if (!workspace) return fail(NSOSX_ERR_INVALID, "scan_fwd_planned: null workspace");
    if (reinterpret_cast<uintptr_t>(workspace) % 256)
        return fail(NSOSX_ERR_INVALID, "scan_fwd_planned: workspace must be 256-byte aligned");
    if (!cu_seqlens || num_seqs <= 0 || num_seqs > 65535 || total_tokens < 0 || H <= 0 || P <= 0 ||
        N <= 0 || N > 64 || G <= 0 || H % G != 0)
        return fail(NSOSX_ERR_INVALID, "scan_fwd_planned: bad shape (N <= 64, G > 0, H % G == 0)");
    if (chunk_tokens > 0 && chunk_tokens < 4)
        return fail(NSOSX_ERR_INVALID, "scan_fwd_planned: chunk_tokens must be >= 4, 0 or -1");
    const int Cn = resolve_chunk(num_seqs, total_tokens, H, P, N, chunk_tokens);
    const int Dm = H * P;
    const ScanWs ws = scan_ws_layout(workspace, num_seqs, total_tokens, Dm, N, Cn);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (Cn == 0) {
        // up to kOrderMax sequences the kernels rank in-workgroup (at most kOrderMax^2
        // compares per wave); beyond, one pre-pass ranks every sequence once
        const bool prepass = num_seqs > kOrderMax && num_seqs <= kOrderPrepassMax;
        if (prepass)
            hipLaunchKernelGGL(scan_order_kernel, dim3((num_seqs + 255) / 256), dim3(256), 0, st,
                               cu_seqlens, num_seqs, total_tokens, ws.order);
        QuadPlan plan{};
        plan.order = prepass ? ws.order : nullptr;
        return scan_fwd_launch(x, x_stride, dt, A_log, a_per_state, B, C, D, z, z_stride,
                               cu_seqlens, num_seqs, total_tokens, H, P, N, G, act_dtype, conv_w,
                               conv_b, conv_width, initial_state, final_state, y, stream, plan);
    }
    const int pg = Dm / G;
    const bool quad_form = N <= 16 && pg % kQuadCh == 0 && (!conv_w || conv_width <= kQuadMaxW);
    const bool lds_form = pg % kScanCh == 0 && (!conv_w || conv_width <= kMaxConvW);
    if (!quad_form && !lds_form)
        return fail(NSOSX_ERR_INVALID, "scan_fwd_planned: the time-chunked scan needs channels "
                                       "per group a multiple of 64 (or of 16 with N <= 16 and "
                                       "conv width <= 4)");
    if ((int64_t)ws.maxc * Dm * N >= ((int64_t)1 << 31) || ws.maxc > 65535)
        return fail(NSOSX_ERR_OVERFLOW, "scan_fwd_planned: too many chunks (at most 65535 and "
                                        "chunks * H*P * N < 2^31): use longer chunks");
    hipLaunchKernelGGL(chunk_plan_kernel, dim3(1), dim3(1024), 0, st, cu_seqlens, num_seqs,
                       total_tokens, Cn, ws.maxc, ws.chunk_cu, ws.seq_start, ws.init_row,
                       ws.state_row, ws.first_chunk);
    // 1. local pass: end states from zero (first chunks from the initial state)
    QuadPlan p1{};
    p1.seq_start = ws.seq_start;
    p1.init_row = ws.init_row;
    p1.sum_dl = ws.sum_dl;
    int rc = scan_fwd_launch(x, x_stride, dt, A_log, a_per_state, B, C, D, nullptr, 0,
                             ws.chunk_cu, ws.maxc, total_tokens, H, P, N, G, act_dtype, conv_w,
                             conv_b, conv_width, initial_state, ws.local, nullptr, stream, p1,
                             true);
    if (rc) return rc;
    // 2. carries across chunk boundaries
    const int64_t threads = (int64_t)num_seqs * Dm * N;
    hipLaunchKernelGGL(chunk_combine_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                       st, ws.first_chunk, num_seqs, Dm, P, N, A_log, a_per_state, ws.local,
                       ws.sum_dl, initial_state, ws.carry);
    // 3. full pass from the carried states
    QuadPlan p3{};
    p3.seq_start = ws.seq_start;
    p3.state_row = ws.state_row;
    return scan_fwd_launch(x, x_stride, dt, A_log, a_per_state, B, C, D, z, z_stride, ws.chunk_cu,
                           ws.maxc, total_tokens, H, P, N, G, act_dtype, conv_w, conv_b,
                           conv_width, ws.carry, final_state, y, stream, p3);
}

extern "C" int nsosx_selective_scan_step(const void* x, const void* dt, const float* A_log,
                                         int a_per_state, const void* B, const void* C,
                                         const float* D, const void* z, int rows, int H, int P,
                                         int N, int G, int act_dtype, float* state, void* y,
                                         void* stream) {
    if (!x || !dt || !A_log || !B || !C || !D || !state || !y)
        return fail(NSOSX_ERR_INVALID, "selective_scan_step: null pointer");
    if (rows <= 0 || H <= 0 || P <= 0 || N <= 0 || N > 64 || G <= 0 || H % G != 0)
        return fail(NSOSX_ERR_INVALID, "selective_scan_step: bad shape");
    if (!valid_dtype(act_dtype)) return fail(NSOSX_ERR_INVALID, "selective_scan_step: bad dtype");
    if (reinterpret_cast<uintptr_t>(state) % 16)
        return fail(NSOSX_ERR_INVALID, "selective_scan_step: state must be 16-byte aligned");
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (N % 4 == 0 && (N / 4 == 1 || N / 4 == 2 || N / 4 == 4 || N / 4 == 8 || N / 4 == 16) &&
        rows <= 65535 * kStepRows) {
        // states of a channel split evenly over the quad: the row-blocked kernel
        const dim3 grid((H * P + 63) / 64, (rows + kStepRows - 1) / kStepRows), block(256);
        // B and C staged per wave when N = 16, they are 8-byte aligned and a wave's 16
        // channels share one group (chosen here: a branch on the alignment inside the kernel
        // would drain its loads)
        const bool vbc = ((reinterpret_cast<uintptr_t>(B) | reinterpret_cast<uintptr_t>(C)) & 7) == 0 &&
                         ((int64_t)H * P / G) % 16 == 0;
#define NSOSX_STEPR(ADT, SPL, GATE, V)                                                             \
    hipLaunchKernelGGL((scan_step_rows_kernel<ADT, SPL, GATE, V>), grid, block, 0, st, x, dt, A_log, \
                       a_per_state, B, C, D, z, rows, H, P, N, G, state, y);
#define NSOSX_STEPR_G(ADT, SPL)                                                   \
    if (SPL == 4 && vbc) {                                                       \
        if (z) { NSOSX_STEPR(ADT, SPL, true, true) } else { NSOSX_STEPR(ADT, SPL, false, true) } \
    } else {                                                                     \
        if (z) { NSOSX_STEPR(ADT, SPL, true, false) } else { NSOSX_STEPR(ADT, SPL, false, false) } \
    }
#define NSOSX_STEPR_S(ADT)                          \
    switch (N / 4) {                                \
        case 1: NSOSX_STEPR_G(ADT, 1) break;        \
        case 2: NSOSX_STEPR_G(ADT, 2) break;        \
        case 4: NSOSX_STEPR_G(ADT, 4) break;        \
        case 8: NSOSX_STEPR_G(ADT, 8) break;        \
        default: NSOSX_STEPR_G(ADT, 16) break;      \
    }
        if (act_dtype == NSOSX_F32) { NSOSX_STEPR_S(NSOSX_F32) } else { NSOSX_STEPR_S(NSOSX_BF16) }
#undef NSOSX_STEPR_S
#undef NSOSX_STEPR_G
#undef NSOSX_STEPR
        return check_launch("selective_scan_step");
    }
    const int64_t lanes = (int64_t)rows * H * P * 4;
    const dim3 grid((unsigned)((lanes + 255) / 256)), block(256);
    const int spl = N <= 4 ? 1 : N <= 8 ? 2 : N <= 16 ? 4 : N <= 32 ? 8 : 16;
#define NSOSX_STEP(ADT, SPL, GATE)                                                              \
    hipLaunchKernelGGL((scan_step_kernel<ADT, SPL, GATE>), grid, block, 0, st, x, dt, A_log,     \
                       a_per_state, B, C, D, z, rows, H, P, N, G, state, y);
#define NSOSX_STEP_G(ADT, SPL) \
    if (z) { NSOSX_STEP(ADT, SPL, true) } else { NSOSX_STEP(ADT, SPL, false) }
#define NSOSX_STEP_S(ADT)                          \
    switch (spl) {                                 \
        case 1: NSOSX_STEP_G(ADT, 1) break;        \
        case 2: NSOSX_STEP_G(ADT, 2) break;        \
        case 4: NSOSX_STEP_G(ADT, 4) break;        \
        case 8: NSOSX_STEP_G(ADT, 8) break;        \
        default: NSOSX_STEP_G(ADT, 16) break;      \
    }
    if (act_dtype == NSOSX_F32) { NSOSX_STEP_S(NSOSX_F32) } else { NSOSX_STEP_S(NSOSX_BF16) }
#undef NSOSX_STEP_S
#undef NSOSX_STEP_G
#undef NSOSX_STEP
    return check_launch("selective_scan_step");
}

// Argument checks and the argument block of the Mamba-2 decode step entries.
static int m2_prepare(const char* what, const void* x, const void* z, const void* B,
                      const void* C, const void* dt, int64_t bcdt_stride, const float* conv_w,
                      const float* conv_b, int conv_width, float* ring, const float* A_log,
                      const float* D, const float* norm_w, float eps, int rows, int H, int P,
                      int N, int G, int act_dtype, float* state, void* y, int8_t* q,
                      float* act_scale, int act_bits, M2StepArgs& a) {
    const std::string w(what);
    if (!x || !z || !B || !C || !dt || !conv_w || !A_log || !D || !state || !y || !q ||
        !act_scale || (conv_width > 1 && !ring))
        return fail(NSOSX_ERR_INVALID, w + ": null pointer");
    if (rows <= 0 || rows > 65535 || H <= 0 || P <= 0 || G <= 0 || H % G != 0 ||
        bcdt_stride <= 0)
        return fail(NSOSX_ERR_INVALID, w + ": bad shape");
    if (!valid_dtype(act_dtype)) return fail(NSOSX_ERR_INVALID, w + ": bad dtype");
    if (!(eps > 0.0f) || !std::isfinite(eps))
        return fail(NSOSX_ERR_INVALID, w + ": eps must be finite and > 0");
    if (act_bits < 2 || act_bits > 8)
        return fail(NSOSX_ERR_INVALID, w + ": act_bits must be in [2, 8]");
    if ((int64_t)H * P > kM2MaxInner || (int64_t)G * N > kM2MaxGS || conv_width < 1 ||
        conv_width > kM2MaxW || !(N == 4 || N == 8 || N == 16 || N == 32 || N == 64))
        return fail(NSOSX_ERR_INVALID,
                    w + ": needs H*P <= 8192, G*N <= 1024, N in {4, 8, 16, 32, 64}, "
                        "1 <= conv_width <= 4");
    if (reinterpret_cast<uintptr_t>(state) % 16)
        return fail(NSOSX_ERR_INVALID, w + ": state must be 16-byte aligned");
    a = M2StepArgs{};
    a.x = x; a.z = z; a.B = B; a.C = C; a.dt = dt; a.bcdt_stride = bcdt_stride;
    a.conv_w = conv_w; a.conv_b = conv_b; a.ring = ring;
    a.a_log = A_log; a.dskip = D; a.norm_w = norm_w; a.eps = eps;
    a.q_max = act_bits <= 2 ? 1.0f : static_cast<float>((1 << (act_bits - 1)) - 1);
    a.H = H; a.P = P; a.N = N; a.G = G; a.W = conv_width;
    a.state = state; a.y = y; a.q = q; a.act_scale = act_scale;
    return NSOSX_OK;
}

static void m2_launch_scan(const M2StepArgs& a, int rows, int act_dtype, hipStream_t st) {
    const dim3 grid((a.H * a.P + 63) / 64, rows);
#define NSOSX_M2(ADT, SPL) \
    hipLaunchKernelGGL((mamba2_step_scan_kernel<ADT, SPL>), grid, dim3(256), 0, st, a);
#define NSOSX_M2_N(ADT)                         \
    switch (a.N) {                              \
        case 4: NSOSX_M2(ADT, 1) break;         \
        case 8: NSOSX_M2(ADT, 2) break;         \
        case 16: NSOSX_M2(ADT, 4) break;        \
        case 32: NSOSX_M2(ADT, 8) break;        \
        default: NSOSX_M2(ADT, 16) break;       \
    }
    if (act_dtype == NSOSX_F32) { NSOSX_M2_N(NSOSX_F32) } else { NSOSX_M2_N(NSOSX_BF16) }
#undef NSOSX_M2_N
#undef NSOSX_M2
}

static void m2_launch_norm(const M2StepArgs& a, int rows, int act_dtype, hipStream_t st) {
    if (act_dtype == NSOSX_F32)
        hipLaunchKernelGGL((mamba2_step_norm_kernel<NSOSX_F32>), dim3(rows), dim3(kM2NormThreads),
                           0, st, a);
    else
        hipLaunchKernelGGL((mamba2_step_norm_kernel<NSOSX_BF16>), dim3(rows),
                           dim3(kM2NormThreads), 0, st, a);
}

extern "C" int nsosx_mamba2_step(const void* x, const void* z, const void* B, const void* C,
                                 const void* dt, int64_t bcdt_stride, const float* conv_w,
                                 const float* conv_b, int conv_width, float* ring,
                                 const float* A_log, const float* D, const float* norm_w,
                                 float eps, int rows, int H, int P, int N, int G, int act_dtype,
                                 float* state, void* y, int8_t* q, float* act_scale,
                                 int act_bits, void* stream) {
    M2StepArgs a;
    const int rc = m2_prepare("mamba2_step", x, z, B, C, dt, bcdt_stride, conv_w, conv_b,
                              conv_width, ring, A_log, D, norm_w, eps, rows, H, P, N, G,
                              act_dtype, state, y, q, act_scale, act_bits, a);
    if (rc) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    m2_launch_scan(a, rows, act_dtype, st);
    m2_launch_norm(a, rows, act_dtype, st);
    return check_launch("mamba2_step");
}

extern "C" int nsosx_mamba2_step_out(const void* x, const void* z, const void* B, const void* C,
                                     const void* dt, int64_t bcdt_stride, const float* conv_w,
                                     const float* conv_b, int conv_width, float* ring,
                                     const float* A_log, const float* D, const float* norm_w,
                                     float eps, int rows, int H, int P, int N, int G,
                                     int act_dtype, float* state, void* y, int8_t* q,
                                     float* act_scale, int act_bits, const uint32_t* out_packed,
                                     float out_weight_scale, int out_features,
                                     const float* out_magnitude, const float* out_bias, void* out,
                                     int out_dtype, void* stream) {
    M2StepArgs a;
    int rc = m2_prepare("mamba2_step_out", x, z, B, C, dt, bcdt_stride, conv_w, conv_b,
                        conv_width, ring, A_log, D, norm_w, eps, rows, H, P, N, G, act_dtype,
                        state, y, q, act_scale, act_bits, a);
    if (rc) return rc;
    const int K = H * P;
    if (!out_packed || !out) return fail(NSOSX_ERR_INVALID, "mamba2_step_out: null pointer");
    if (out_features <= 0 || K % 16 != 0 || !valid_dtype(out_dtype) ||
        !(out_weight_scale > 0.0f) || !std::isfinite(out_weight_scale))
        return fail(NSOSX_ERR_INVALID,
                    "mamba2_step_out: need out_features > 0, H*P % 16 == 0, a finite weight "
                    "scale > 0");
    hipStream_t st = static_cast<hipStream_t>(stream);
    m2_launch_scan(a, rows, act_dtype, st);
    if (mamba2_norm_gemv_ok(rows, K) && (reinterpret_cast<uintptr_t>(out_packed) & 15) == 0) {
        rc = check_launch("mamba2_step_out");
        if (rc) return rc;
        return launch_mamba2_norm_gemv(a, act_dtype, out_packed, out_weight_scale, out_features,
                                       out_magnitude, out_bias, out, out_dtype, st);
    }
    m2_launch_norm(a, rows, act_dtype, st);
    rc = check_launch("mamba2_step_out");
    if (rc) return rc;
    return nsosx_ternary_gemm(q, act_scale, out_packed, out_weight_scale, rows, K, out_features,
                              out_magnitude, out_bias, out, out_dtype, nullptr, stream);
}

extern "C" int nsosx_conv1d_causal(const void* in, int in_dtype, int64_t in_stride,
                                   const float* weight, const float* bias,
                                   const int32_t* cu_seqlens, int num_seqs, int total_tokens,
                                   int channels, int width, int apply_silu, void* out,
                                   int out_dtype, void* stream) {
    if (!in || !weight || !cu_seqlens || !out)
        return fail(NSOSX_ERR_INVALID, "conv1d_causal: null pointer");
    if (num_seqs <= 0 || total_tokens < 0 || channels <= 0 || channels > 65535 * 256 ||
        width <= 0 || width > 64 || in_stride < channels)
        return fail(NSOSX_ERR_INVALID, "conv1d_causal: bad shape");
    if (!valid_dtype(in_dtype) || !valid_dtype(out_dtype))
        return fail(NSOSX_ERR_INVALID, "conv1d_causal: bad dtype");
    if (total_tokens == 0) return NSOSX_OK;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int64_t elems = (int64_t)total_tokens * channels;
    if (elems > (int64_t)256 * 0x7FFFFFFF) return fail(NSOSX_ERR_OVERFLOW, "conv1d_causal: too large");
    const dim3 grid(static_cast<unsigned>((elems + 255) / 256)), block(256);
#define NSOSX_CONV(I, O)                                                                        \
    hipLaunchKernelGGL((conv1d_kernel<I, O>), grid, block, 0, st, in, in_stride, weight, bias,    \
                       cu_seqlens, num_seqs, total_tokens, channels, width, apply_silu, out);
    if (in_dtype == NSOSX_F32) {
        if (out_dtype == NSOSX_F32) { NSOSX_CONV(NSOSX_F32, NSOSX_F32) } else { NSOSX_CONV(NSOSX_F32, NSOSX_BF16) }
    } else {
        if (out_dtype == NSOSX_F32) { NSOSX_CONV(NSOSX_BF16, NSOSX_F32) } else { NSOSX_CONV(NSOSX_BF16, NSOSX_BF16) }
    }
#undef NSOSX_CONV
    return check_launch("conv1d_causal");
}
