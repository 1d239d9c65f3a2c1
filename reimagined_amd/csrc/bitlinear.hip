// BitLinear hot path on gfx950: activation quantization, the packed-weight
// streaming GEMV (decode) and the int8-MFMA GEMM (prefill, grouped experts).
//
// Reference semantics (OXN/nsos/ of vitorGgC569/reimagined):
//   quantization  src/bitlinear.cpp:240-291, src/bitlinear_quantize_avx2.cpp:65-103
//   RMS_PERI norm src/bitlinear.cpp:460-466, src/tensor.cpp:3455-3492
//   GEMM + affine src/bitnet_adapter_avx2.cpp:52-158
//   packed format src/bitnet_adapter.cpp:570-606
#include "common.hpp"
#include "mamba2_step.hpp"

#include <algorithm>
#include <cmath>

namespace nsosx {

// ===========================================================================
// RMS_PERI: inv[r] = 1 / sqrt(sum_sq / K + eps) with the float sum taken in
// index order (rounded square, then add) as the reference's sequential loop
// does; a remainder of K % 4 elements is accumulated with fma, which is how
// that loop is compiled.  The sum is a chain of K dependent adds, so the
// parallelism is across rows: lane = row, each lane streaming its own row
// with 16-byte loads (eight bf16 or four f32 values per load, four loads in
// flight).
// ===========================================================================
template <int DT>
__device__ __forceinline__ void load16_f32(const char* p, float v[DT == NSOSX_F32 ? 4 : 8]) {
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    if constexpr (DT == NSOSX_F32) {
        v[0] = __uint_as_float(a.x); v[1] = __uint_as_float(a.y);
        v[2] = __uint_as_float(a.z); v[3] = __uint_as_float(a.w);
    } else {
        const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = __uint_as_float(w[i] << 16);
            v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    }
}

template <int DT, bool VEC>
__global__ __launch_bounds__(64) void rms_inv_kernel(const void* __restrict__ x, int M, int K,
                                                     float eps, float* __restrict__ inv) {
    const int row = blockIdx.x * 64 + threadIdx.x;
    if (row >= M) return;
    constexpr int ES = DT == NSOSX_F32 ? 4 : 2;
    constexpr int PER = 16 / ES;  // elements per 16-byte load
    const char* base = static_cast<const char*>(x) + (int64_t)row * K * ES;
    const int body = K & ~3;
    float sum = 0.0f;
    int k = 0;
    if (VEC) {
        constexpr int U = 4;  // loads in flight
        for (; k + U * PER <= body; k += U * PER) {
            float v[U][PER];
#pragma unroll
            for (int u = 0; u < U; ++u) load16_f32<DT>(base + (int64_t)(k + u * PER) * ES, v[u]);
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int j = 0; j < PER; ++j) sum = __fadd_rn(sum, __fmul_rn(v[u][j], v[u][j]));
        }
    }
    for (; k < K; ++k) {
        const float v = load_act<DT>(x, (int64_t)row * K + k);
        if (k < body) sum = __fadd_rn(sum, __fmul_rn(v, v));
        else sum = __fmaf_rn(v, v, sum);
    }
    const float mean = __fdiv_rn(sum, static_cast<float>(K > 1 ? K : 1));
    // sqrtf is IEEE-rounded under -fhip-fp32-correctly-rounded-divide-sqrt;
    // __fsqrt_rn is not (it maps to the native approximation)
    inv[row] = __fdiv_rn(1.0f, sqrtf(__fadd_rn(mean, eps)));
}

// Many rows, rows of a multiple of kRmsDepth tiles: the same in-order sums,
// lane = row, with the rows coming in through LDS.  A one-wave workgroup owns
// 64 rows and streams them in column tiles of kRmsTileBytes per row: a tile is
// read with 1 KB loads (whole 128-byte lines, where lane-per-row loads touch 64
// lines per instruction), kRmsDepth tiles in flight in registers, and passed
// through a double-buffered LDS slice from which each lane sums its own row.
// LDS operations of one wave complete in order, so no barrier is needed.
constexpr int kRmsTileBytes = 128;                    // bytes of a row per tile
constexpr int kRmsRowPitch = kRmsTileBytes + 16;      // padded LDS row (bank spread)
constexpr int kRmsDepth = 4;                          // tiles in flight

template <int DT>
__global__ __launch_bounds__(64) void rms_inv_tiled_kernel(const void* __restrict__ x, int M,
                                                           int K, float eps,
                                                           float* __restrict__ inv) {
    __shared__ __align__(16) char s_tile[2][64 * kRmsRowPitch];
    constexpr int ES = DT == NSOSX_F32 ? 4 : 2;
    constexpr int PER = 16 / ES;                      // elements per 16 bytes
    constexpr int TE = kRmsTileBytes / ES;            // elements of a row per tile
    const int lane = threadIdx.x;
    const int row0 = blockIdx.x * 64;
    const int64_t row_bytes = (int64_t)K * ES;
    const char* xb = static_cast<const char*>(x);
    const int tiles = K / TE;
    // load j (0..7) of a tile: row 8 j + lane / 8, 16-byte piece lane % 8; rows past M
    // re-read the last row and tiles past the end the last tile (never used)
    const char* src[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
        src[j] = xb + min(row0 + 8 * j + (lane >> 3), M - 1) * row_bytes + (lane & 7) * 16;
    uint4 buf[kRmsDepth][8];
    auto load_tile = [&](int t, uint4 (&b)[8]) {
        const int64_t off = (int64_t)min(t, tiles - 1) * kRmsTileBytes;
#pragma unroll
        for (int j = 0; j < 8; ++j) b[j] = load_stream16(reinterpret_cast<const uint32_t*>(src[j] + off));
    };
#pragma unroll
    for (int d = 0; d < kRmsDepth; ++d) load_tile(d, buf[d]);
    float sum = 0.0f;
    for (int t0 = 0; t0 < tiles; t0 += kRmsDepth) {
        // tiles is a multiple of kRmsDepth (host check): straight-line code, so the
        // loads stay in flight across tiles
#pragma unroll
        for (int d = 0; d < kRmsDepth; ++d) {
            const int t = t0 + d;
            char* slot = s_tile[d & 1];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                *reinterpret_cast<uint4*>(slot + (8 * j + (lane >> 3)) * kRmsRowPitch +
                                          (lane & 7) * 16) = buf[d][j];
            load_tile(t + kRmsDepth, buf[d]);
            const char* my = slot + lane * kRmsRowPitch;
#pragma unroll
            for (int p = 0; p < kRmsTileBytes / 16; ++p) {
                float v[PER];
                load16_f32<DT>(my + p * 16, v);
#pragma unroll
                for (int j = 0; j < PER; ++j) sum = __fadd_rn(sum, __fmul_rn(v[j], v[j]));
            }
        }
    }
    const int row = row0 + lane;
    if (row >= M) return;
    const float mean = __fdiv_rn(sum, static_cast<float>(K));
    inv[row] = __fdiv_rn(1.0f, sqrtf(__fadd_rn(mean, eps)));
}

// The same sums for fewer rows, where the tiled kernel's one wave per 64 rows
// leaves most SIMDs idle and runs the whole row's convert / square / add chain
// alone.  Here two producer waves (rows 0-31 and 32-63 of the group)
// load the column tiles (1 KB loads, kRmsPcDepth tiles in flight), convert and
// square them, and write the rounded squares to a double-buffered LDS tile in
// row order; a third wave (lane = row) adds them in order, one tile behind,
// with one barrier per tile.  Same operations in the same order, so the same
// bits as rms_inv_tiled_kernel.
constexpr int kRmsPcPitch = 64 + 4;  // floats per LDS row (one tile of 64 squares + pad)
constexpr int kRmsPcDepth = 8;       // tiles in flight per producer wave

// NP producer waves of 32 rows each (the group is 32 NP rows): 2, or 1 where
// two-wave groups would leave the CUs with fewer than two groups each.
template <int DT, int NP>
__global__ __launch_bounds__((NP + 1) * 64) void rms_inv_pc_kernel(const void* __restrict__ x,
                                                                   int M, int K, float eps,
                                                                   float* __restrict__ inv) {
    constexpr int ES = DT == NSOSX_F32 ? 4 : 2;
    constexpr int PER = 16 / ES;            // elements per 16-byte piece
    constexpr int TE = kRmsTileBytes / ES;  // elements of a row per tile
    __shared__ __align__(16) float s_sq[2][32 * NP * kRmsPcPitch];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int row0 = blockIdx.x * 32 * NP;
    const int tiles = K / TE;
    const int64_t row_bytes = (int64_t)K * ES;
    if (wave < NP) {
        // load j (0..3) of a tile: row 32 wave + 8 j + lane / 8, 16-byte piece lane % 8;
        // rows past M re-read the last row and tiles past the end the last tile
        const char* src[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            src[j] = static_cast<const char*>(x) +
                     min(row0 + 32 * wave + 8 * j + (lane >> 3), M - 1) * row_bytes + (lane & 7) * 16;
        uint4 buf[kRmsPcDepth][4];
        auto load_tile = [&](int t, uint4 (&b)[4]) {
            const int64_t off = (int64_t)min(t, tiles - 1) * kRmsTileBytes;
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = load_stream16(reinterpret_cast<const uint32_t*>(src[j] + off));
        };
#pragma unroll
        for (int d = 0; d < kRmsPcDepth; ++d) load_tile(d, buf[d]);
        // tiles is a multiple of kRmsPcDepth (host check): straight-line steady state, the
        // loads past the end clamped to the last tile
        for (int t0 = 0; t0 < tiles; t0 += kRmsPcDepth) {
#pragma unroll
            for (int d = 0; d < kRmsPcDepth; ++d) {
                const int t = t0 + d;
                float* dst = s_sq[t & 1];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint4 a = buf[d][j];
                    float v[PER];
                    if constexpr (DT == NSOSX_F32) {
                        v[0] = __uint_as_float(a.x); v[1] = __uint_as_float(a.y);
                        v[2] = __uint_as_float(a.z); v[3] = __uint_as_float(a.w);
                    } else {
                        const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            v[2 * i] = __uint_as_float(w[i] << 16);
                            v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
                        }
                    }
                    float* q = dst + (32 * wave + 8 * j + (lane >> 3)) * kRmsPcPitch + (lane & 7) * PER;
#pragma unroll
                    for (int i = 0; i < PER; i += 4)
                        *reinterpret_cast<float4*>(q + i) =
                            make_float4(__fmul_rn(v[i], v[i]), __fmul_rn(v[i + 1], v[i + 1]),
                                        __fmul_rn(v[i + 2], v[i + 2]), __fmul_rn(v[i + 3], v[i + 3]));
                }
                load_tile(t + kRmsPcDepth, buf[d]);
                __syncthreads();
            }
        }
    } else {
        // one tile behind the producers: tile t - 1 during their tile t, the last after the loop
        float sum = 0.0f;
        // (with one producer wave, lanes 32-63 repeat row 31's sums and store nothing)
        const int off = min(lane, 32 * NP - 1) * kRmsPcPitch;
        auto add_tile = [&](int t) {
            const float* my = s_sq[t & 1] + off;
#pragma unroll
            for (int i = 0; i < TE; i += 4) {
                const float4 v = *reinterpret_cast<const float4*>(my + i);
                sum = __fadd_rn(sum, v.x);
                sum = __fadd_rn(sum, v.y);
                sum = __fadd_rn(sum, v.z);
                sum = __fadd_rn(sum, v.w);
            }
        };
        for (int t = 0; t < tiles; ++t) {
            if (t > 0) add_tile(t - 1);
            __syncthreads();
        }
        add_tile(tiles - 1);
        const int row = row0 + lane;
        if (lane < 32 * NP && row < M) {
            const float mean = __fdiv_rn(sum, static_cast<float>(K));
            inv[row] = __fdiv_rn(1.0f, sqrtf(__fadd_rn(mean, eps)));
        }
    }
}

// Few rows (decode): a workgroup per row stages the row in LDS with coalesced
// 16-byte loads, then one lane takes the in-order sum from LDS, so the row's
// load latency is paid once instead of once per four loads.  K <= 8192.
constexpr int kRmsSmallMaxK = 8192;

template <int DT>
__global__ __launch_bounds__(256) void rms_inv_small_kernel(const void* __restrict__ x, int K,
                                                            float eps, float* __restrict__ inv) {
    __shared__ __align__(16) float s_row[kRmsSmallMaxK];
    const int row = blockIdx.x;
    const int64_t base = (int64_t)row * K;
    const int body = K & ~3;
    // body elements as their rounded squares (the lane walking the row only adds),
    // the K % 4 tail as values for the fused multiply-adds
    for (int k = threadIdx.x; k < K; k += 256) {
        const float v = load_act<DT>(x, base + k);
        s_row[k] = k < body ? __fmul_rn(v, v) : v;
    }
    __syncthreads();
    if (threadIdx.x != 0) return;
    float sum = 0.0f;
#pragma unroll 8
    for (int k = 0; k < body; k += 4) {
        const float4 v = *reinterpret_cast<const float4*>(s_row + k);
        sum = __fadd_rn(sum, v.x);
        sum = __fadd_rn(sum, v.y);
        sum = __fadd_rn(sum, v.z);
        sum = __fadd_rn(sum, v.w);
    }
    for (int k = body; k < K; ++k) sum = __fmaf_rn(s_row[k], s_row[k], sum);
    const float mean = __fdiv_rn(sum, static_cast<float>(K > 1 ? K : 1));
    inv[row] = __fdiv_rn(1.0f, sqrtf(__fadd_rn(mean, eps)));
}

// ===========================================================================
// Per-row absmax quantization, one wave per row.
//   m = max|x|; s = q_max / (m + 1e-8f); act_scale = (m + 1e-8f) / q_max;
//   code = round(x * s), ties to even for the first K & ~7 elements (the
//   AVX2 body) and half away from zero for the K % 8 tail (std::round);
//   int8 = clamp(code, -127, 127).
// VEC: K % 8 == 0, every row 16-byte aligned -> 8 elements per lane-load,
// the row kept in registers between the two passes when K <= 4096.
// ===========================================================================
template <int DT>
__device__ __forceinline__ void load8(const void* x, int64_t off, float v[8]) {
    if constexpr (DT == NSOSX_F32) {
        const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(x) + off);
        const float4 a = p[0], b = p[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
        const uint4 a = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + off);
        const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = __uint_as_float(w[i] << 16);
            v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    }
}


// ===========================================================================
// Few rows with RMS_PERI (decode): the RMS pass and the quantization in one
// launch.  A workgroup per row keeps the row in registers (8 elements per
// thread and 2048-element chunk, K % 8 == 0, K <= 4096) and in LDS as floats;
// lane 0 takes the in-order sum from LDS, the workgroup the absmax of x * inv
// and the codes, with the operations of rms_inv_small_kernel and
// quantize_rows_vec_kernel<DT, true> (so the same bits).
// ===========================================================================
constexpr int kQSmallMaxK = 4096;

// One row by a 256-thread workgroup (K % 8 == 0, K <= 4096): with RMS, the squares
// to s_row and the in-order sum by lane 0 (rms_inv_small_kernel's operations), then
// the absmax of x * inv (x without RMS) and the codes, as quantize_rows_vec_kernel;
// the codes to qrow and act_scale / inv (RMS) to *scale_out / *inv_out (global
// memory or LDS).
template <int DT, bool RMS>
__device__ __forceinline__ void quantize_row_wg(const void* __restrict__ x, int64_t base, int K,
                                                float q_max, float eps, float* s_row,
                                                float* s_red, int8_t* qrow, float* scale_out,
                                                float* inv_out) {
    const int tid = threadIdx.x;
    float v[2][8];
    // the squares (each rounded on its own, as in the in-order sum) go to LDS, so the
    // one lane that walks the row only adds: a chain of K dependent adds
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const int e0 = (c * 256 + tid) * 8;
        if (e0 < K) {
            load8<DT>(x, base + e0, v[c]);
            if (RMS) {
                float q[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) q[j] = __fmul_rn(v[c][j], v[c][j]);
                *reinterpret_cast<float4*>(s_row + e0) = make_float4(q[0], q[1], q[2], q[3]);
                *reinterpret_cast<float4*>(s_row + e0 + 4) = make_float4(q[4], q[5], q[6], q[7]);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) v[c][j] = 0.0f;
        }
    }
    if (RMS) {
        __syncthreads();
        if (tid == 0) {
            float sum = 0.0f;
#pragma unroll 8
            for (int k = 0; k < K; k += 4) {
                const float4 a = *reinterpret_cast<const float4*>(s_row + k);
                sum = __fadd_rn(sum, a.x);
                sum = __fadd_rn(sum, a.y);
                sum = __fadd_rn(sum, a.z);
                sum = __fadd_rn(sum, a.w);
            }
            const float mean = __fdiv_rn(sum, static_cast<float>(K));
            const float inv = __fdiv_rn(1.0f, sqrtf(__fadd_rn(mean, eps)));
            s_red[4] = inv;
            if (inv_out) *inv_out = inv;
        }
        __syncthreads();
        const float inv = s_red[4];
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int j = 0; j < 8; ++j) v[c][j] = __fmul_rn(v[c][j], inv);
    }
    float m = 0.0f;
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(v[c][j]));
    m = wave_max(m);
    if ((tid & 63) == 0) s_red[tid >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    const float denom = __fadd_rn(m, 1e-8f);
    const float sc = __fdiv_rn(q_max, denom);
    if (tid == 0) *scale_out = __fdiv_rn(denom, q_max);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const int e0 = (c * 256 + tid) * 8;
        if (e0 < K) {
            float code[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) code[j] = clamp127(rintf(__fmul_rn(v[c][j], sc)));
            uint2 out;
            out.x = pack4_i8(code[0], code[1], code[2], code[3]);
            out.y = pack4_i8(code[4], code[5], code[6], code[7]);
            *reinterpret_cast<uint2*>(qrow + e0) = out;
        }
    }
}

template <int DT>
__global__ __launch_bounds__(256) void quantize_small_rms_kernel(const void* __restrict__ x,
                                                                 int K, float q_max, float eps,
                                                                 float* __restrict__ rms_inv,
                                                                 int8_t* __restrict__ q,
                                                                 float* __restrict__ act_scale) {
    __shared__ __align__(16) float s_row[kQSmallMaxK];
    __shared__ float s_red[5];
    const int row = blockIdx.x;
    quantize_row_wg<DT, true>(x, (int64_t)row * K, K, q_max, eps, s_row, s_red,
                              q + (int64_t)row * K, act_scale + row, rms_inv + row);
}

template <int DT, bool RMS>
__global__ __launch_bounds__(256) void quantize_rows_vec_kernel(
    const void* __restrict__ x, int M, int K, float q_max, const float* __restrict__ rms_inv,
    int8_t* __restrict__ q, float* __restrict__ act_scale) {
    constexpr int kMaxChunks = 8;  // 8 chunks x 8 elements x 64 lanes = 4096 (K <= 4096)
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    const int64_t base = static_cast<int64_t>(row) * K;
    const float inv = RMS ? rms_inv[row] : 1.0f;
    float v[kMaxChunks][8];
    float m = 0.0f;
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) {
        const int e0 = (c * kWave + lane) * 8;
        if (e0 < K) {
            load8<DT>(x, base + e0, v[c]);
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) v[c][j] = 0.0f;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (RMS) v[c][j] = __fmul_rn(v[c][j], inv);
            m = fmaxf(m, fabsf(v[c][j]));
        }
    }
    m = wave_max(m);
    const float denom = __fadd_rn(m, 1e-8f);
    const float s = __fdiv_rn(q_max, denom);
    if (lane == 0) act_scale[row] = __fdiv_rn(denom, q_max);
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) {
        const int e0 = (c * kWave + lane) * 8;
        if (e0 < K) {
            float code[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) code[j] = clamp127(rintf(__fmul_rn(v[c][j], s)));
            uint2 out;
            out.x = pack4_i8(code[0], code[1], code[2], code[3]);
            out.y = pack4_i8(code[4], code[5], code[6], code[7]);
            *reinterpret_cast<uint2*>(q + base + e0) = out;
        }
    }
}

// Many rows with K = CH x 512: a wave quantizes RPW = 8 / CH rows and issues
// all RPW x CH chunk loads (8 elements per lane each) before it uses any, so a
// wave keeps 8 KB of bf16 in flight where one row per wave kept 1-2 KB (the
// row-per-wave kernel is latency-bound at ~3.9 TB/s).  The float operations
// are those of quantize_rows_vec_kernel (x * inv is formed again for the codes,
// the same product), so the same bits.
template <int DT, bool RMS, int CH>
__global__ __launch_bounds__(256) void quantize_rows_multi_kernel(
    const void* __restrict__ x, int M, float q_max, const float* __restrict__ rms_inv,
    int8_t* __restrict__ q, float* __restrict__ act_scale) {
    constexpr int RPW = 8 / CH;
    constexpr int K = CH * kWave * 8;
    constexpr int ES = DT == NSOSX_F32 ? 4 : 2;  // bytes per element
    constexpr int NW = ES / 2;                   // 16-byte words per 8-element chunk
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW;
    if (row0 >= M) return;
    uint4 raw[RPW][CH][NW];
    float invs[RPW];  // fetched with the rows: no load waits between one row's codes and the next
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int row = min(row0 + r, M - 1);  // rows past M re-read row M - 1 and are not stored
        invs[r] = RMS ? rms_inv[row] : 1.0f;
        const char* src = static_cast<const char*>(x) + ((int64_t)row * K + lane * 8) * ES;
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int w = 0; w < NW; ++w)
                raw[r][c][w] = *reinterpret_cast<const uint4*>(src + c * (kWave * 8 * ES) + w * 16);
    }
    auto unpack = [&](const uint4 (&u)[NW], float v[8]) {
        if constexpr (DT == NSOSX_F32) {
            const uint32_t w[8] = {u[0].x, u[0].y, u[0].z, u[0].w, u[NW - 1].x, u[NW - 1].y,
                                   u[NW - 1].z, u[NW - 1].w};
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = __uint_as_float(w[j]);
        } else {
            const uint32_t w[4] = {u[0].x, u[0].y, u[0].z, u[0].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[2 * i] = __uint_as_float(w[i] << 16);
                v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
            }
        }
    };
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int row = row0 + r;
        const float inv = invs[r];
        float m = 0.0f;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            float v[8];
            unpack(raw[r][c], v);
#pragma unroll
            for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(RMS ? __fmul_rn(v[j], inv) : v[j]));
        }
        m = wave_max(m);
        if (row >= M) break;
        const float denom = __fadd_rn(m, 1e-8f);
        const float sc = __fdiv_rn(q_max, denom);
        if (lane == 0) act_scale[row] = __fdiv_rn(denom, q_max);
        int8_t* dst = q + (int64_t)row * K + lane * 8;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            float v[8], code[8];
            unpack(raw[r][c], v);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                code[j] = clamp127(rintf(__fmul_rn(RMS ? __fmul_rn(v[j], inv) : v[j], sc)));
            *reinterpret_cast<uint2*>(dst + c * kWave * 8) =
                make_uint2(pack4_i8(code[0], code[1], code[2], code[3]),
                           pack4_i8(code[4], code[5], code[6], code[7]));
        }
    }
}

template <int DT, bool RMS, int CH>
static void launch_quantize_multi(const void* x, int M, float qm, const float* rms_ws, int8_t* q,
                                  float* act_scale, hipStream_t st) {
    const int rows_per_wg = 4 * (8 / CH);
    hipLaunchKernelGGL((quantize_rows_multi_kernel<DT, RMS, CH>), dim3((M + rows_per_wg - 1) / rows_per_wg),
                       dim3(256), 0, st, x, M, qm, rms_ws, q, act_scale);
}

// Any K: element-wise loads, the ties-to-even body / half-away tail split.
template <int DT, bool RMS>
__global__ __launch_bounds__(256) void quantize_rows_generic_kernel(
    const void* __restrict__ x, int M, int K, float q_max, const float* __restrict__ rms_inv,
    int8_t* __restrict__ q, float* __restrict__ act_scale) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    const int64_t base = static_cast<int64_t>(row) * K;
    const float inv = RMS ? rms_inv[row] : 1.0f;
    float m = 0.0f;
    for (int j = lane; j < K; j += kWave) {
        float t = load_act<DT>(x, base + j);
        if (RMS) t = __fmul_rn(t, inv);
        m = fmaxf(m, fabsf(t));
    }
    m = wave_max(m);
    const float denom = __fadd_rn(m, 1e-8f);
    const float s = __fdiv_rn(q_max, denom);
    if (lane == 0) act_scale[row] = __fdiv_rn(denom, q_max);
    const int body = K & ~7;
    for (int j = lane; j < K; j += kWave) {
        float t = load_act<DT>(x, base + j);
        if (RMS) t = __fmul_rn(t, inv);
        const float val = __fmul_rn(t, s);
        const float code = j < body ? rintf(val) : roundf(val);
        q[base + j] = static_cast<int8_t>(static_cast<int>(clamp127(code)));
    }
}

static float q_max_for_bits(int bits) {
    if (bits <= 2) return 1.0f;
    return static_cast<float>((1 << (bits - 1)) - 1);
}

// inv[m] = 1 / sqrt(sum_k x[m,k]^2 / K + eps) with the reference's in-order sum
// (Tensor::rmsnorm, src/tensor.cpp:3455-3492): the kernel is picked by shape.
template <int DT>
static void launch_rms_inv_t(const void* x, int M, int K, float eps, float* inv, hipStream_t st) {
    const int elem = DT == NSOSX_F32 ? 4 : 2;
    if (M <= 1024 && K <= kRmsSmallMaxK) {
        hipLaunchKernelGGL((rms_inv_small_kernel<DT>), dim3(M), dim3(256), 0, st, x, K, eps, inv);
    } else if (((int64_t)K * elem) % (kRmsTileBytes * kRmsDepth) == 0 &&
               reinterpret_cast<uintptr_t>(x) % 16 == 0) {
        // fewer than 512 groups of 64 rows: the producer / consumer form (config 5's 16384
        // hidden rows of 4096 in 33 us; its 8192 input rows of 1024, 128 groups, as 256 groups
        // of 32 rows); with more groups the one-wave form streams faster (config 4: 40796 rows
        // of 1024 / 2048, 3 / 6 us less)
        if ((M + 63) / 64 < 512 && ((int64_t)K * elem) % (kRmsTileBytes * kRmsPcDepth) == 0) {
            if ((M + 63) / 64 <= 128)
                hipLaunchKernelGGL((rms_inv_pc_kernel<DT, 1>), dim3((M + 31) / 32), dim3(128), 0, st,
                                   x, M, K, eps, inv);
            else
                hipLaunchKernelGGL((rms_inv_pc_kernel<DT, 2>), dim3((M + 63) / 64), dim3(192), 0, st,
                                   x, M, K, eps, inv);
        }
        else
            hipLaunchKernelGGL((rms_inv_tiled_kernel<DT>), dim3((M + 63) / 64), dim3(64), 0, st, x,
                               M, K, eps, inv);
    } else {
        const bool rvec = ((int64_t)K * elem) % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
        if (rvec)
            hipLaunchKernelGGL((rms_inv_kernel<DT, true>), dim3((M + 63) / 64), dim3(64), 0, st, x,
                               M, K, eps, inv);
        else
            hipLaunchKernelGGL((rms_inv_kernel<DT, false>), dim3((M + 63) / 64), dim3(64), 0, st,
                               x, M, K, eps, inv);
    }
}

void launch_rms_inv(const void* x, int dtype, int M, int K, float eps, float* inv,
                    hipStream_t st) {
    if (dtype == NSOSX_F32) launch_rms_inv_t<NSOSX_F32>(x, M, K, eps, inv, st);
    else launch_rms_inv_t<NSOSX_BF16>(x, M, K, eps, inv, st);
}

template <int DT>
static int launch_quantize(const void* x, int M, int K, int bits, int rms_input, int8_t* q,
                           float* act_scale, float* rms_ws, hipStream_t st) {
    const float qm = q_max_for_bits(bits);
    const int elem = DT == NSOSX_F32 ? 4 : 2;
    if (rms_input && M <= 1024 && K % 8 == 0 && K <= kQSmallMaxK &&
        reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(q) % 8 == 0) {
        hipLaunchKernelGGL((quantize_small_rms_kernel<DT>), dim3(M), dim3(256), 0, st, x, K, qm,
                           1e-6f, rms_ws, q, act_scale);
        return check_launch("quantize_act");
    }
    if (rms_input) launch_rms_inv_t<DT>(x, M, K, 1e-6f, rms_ws, st);
    if ((K == 512 || K == 1024 || K == 2048 || K == 4096) && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
        reinterpret_cast<uintptr_t>(q) % 8 == 0) {
#define NSOSX_QMULTI(CH)                                                                   \
    (rms_input ? launch_quantize_multi<DT, true, CH>(x, M, qm, rms_ws, q, act_scale, st)   \
               : launch_quantize_multi<DT, false, CH>(x, M, qm, rms_ws, q, act_scale, st))
        if (K == 512) NSOSX_QMULTI(1);
        else if (K == 1024) NSOSX_QMULTI(2);
        else if (K == 2048) NSOSX_QMULTI(4);
        else NSOSX_QMULTI(8);
#undef NSOSX_QMULTI
        return check_launch("quantize_act");
    }
    const bool vec = (K % 8 == 0) && K <= 4096 && (reinterpret_cast<uintptr_t>(x) % 16 == 0) &&
                     (reinterpret_cast<uintptr_t>(q) % 8 == 0) && ((int64_t)K * elem) % 16 == 0;
    const dim3 grid((M + 3) / 4), block(256);
    if (vec) {
        if (rms_input)
            hipLaunchKernelGGL((quantize_rows_vec_kernel<DT, true>), grid, block, 0, st, x, M, K,
                               qm, rms_ws, q, act_scale);
        else
            hipLaunchKernelGGL((quantize_rows_vec_kernel<DT, false>), grid, block, 0, st, x, M, K,
                               qm, rms_ws, q, act_scale);
    } else {
        if (rms_input)
            hipLaunchKernelGGL((quantize_rows_generic_kernel<DT, true>), grid, block, 0, st, x, M,
                               K, qm, rms_ws, q, act_scale);
        else
            hipLaunchKernelGGL((quantize_rows_generic_kernel<DT, false>), grid, block, 0, st, x, M,
                               K, qm, rms_ws, q, act_scale);
    }
    return check_launch("quantize_act");
}

// ===========================================================================
// Streaming GEMV (M <= 8).  A row of W is K/16 words; a lane takes a chunk
// of 4 words (64 weights, one 16-byte load) and LPR lanes share a row, LPR
// the smallest power of two >= K/64 (capped at 64), so one wave-load covers
// 64/LPR rows.  The lane's activation chunk is byte-transposed into the
// unpack order once and reused for every row the wave visits; partial sums
// meet in a butterfly over the row's lanes.
// ===========================================================================
struct GemvProblem {
    const uint32_t* packed;
    const float* mag;
    const float* bias;
    float ws;
    int N;
    int K;
};

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

// A group of a grouped GEMV with M >= 2 rows that the skinny MFMA body takes:
// K = 1024 or 2048 (its fragments fit the launch's 64 KB of LDS) and whole
// 4-output vectors (N % 4 == 0, 16-byte aligned rows).
__device__ __forceinline__ bool skinny_group(const nsosx_linear_view& v, const void* yb) {
    return (v.inputs == 1024 || v.inputs == 2048) && (v.outputs & 3) == 0 &&
           (reinterpret_cast<uintptr_t>(yb) & 15) == 0;
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
    const nsosx_linear_view v = views[view_sel ? view_sel[g] : g];
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

// ===========================================================================
// int8 MFMA GEMM.  The packed weight rows are the MFMA's A operand (rows i =
// output columns n) and the activation rows its B operand (columns j = tokens
// m), so each lane's four accumulators are four consecutive n of one token.
// Block tile 256 (n) x 128 (m) x 64 (k), 4 waves in 2x2, each wave 128 x 64
// = 8 x 4 tiles of v_mfma_i32_16x16x64_i8.  Weights stay 2-bit in LDS (4 KB
// per k step) and are expanded to int8 in registers right before the MFMA;
// activation rows are byte-transposed into the same k order on their way to
// LDS (row stride 80 bytes: conflict-free 16-byte reads).  Two LDS stages,
// the next k step's global loads in flight during the current MFMAs.
// GATHER: token rows come through perm[] (MoE slots -> token rows); the m
// range of each expert is its segment [offsets[e], offsets[e+1]).
// ===========================================================================
typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kBN = 256, kBM = 128, kBK = 64;
constexpr int kXStride = 80;  // bytes per activation row in LDS

struct GemmProblem {
    const uint32_t* packed;
    const float* mag;
    const float* bias;
    float ws;
    int N;
    int K;
};

template <int YDT, bool ACC_OUT, bool GATHER, bool SQRELU>
__device__ __forceinline__ void gemm_tile(const GemmProblem& pb, const int8_t* __restrict__ q,
                                          const float* __restrict__ act_scale,
                                          const int32_t* __restrict__ perm, int seg_begin,
                                          int seg_rows, int n0, int m0, void* y,
                                          int32_t* acc_out, char* smem) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wn = wave & 1, wm = wave >> 1;
    const int W16 = pb.K >> 4;
    const int KT = (pb.K + kBK - 1) / kBK;
    const bool waligned = (W16 & 3) == 0;

    uint32_t* wlds[2] = {reinterpret_cast<uint32_t*>(smem),
                         reinterpret_cast<uint32_t*>(smem + kBN * 16)};
    char* xlds[2] = {smem + 2 * kBN * 16, smem + 2 * kBN * 16 + kBM * kXStride};

    // global -> register staging: one weight row chunk and two activation chunks per thread
    const int wrow = n0 + tid;
    const uint32_t* wsrc = pb.packed + (int64_t)wrow * W16;
    int xrow_src[2];
    bool xrow_ok[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int ml = (tid >> 2) + 64 * i;
        const int m = m0 + ml;
        xrow_ok[i] = m < seg_rows;
        int src = seg_begin + m;
        if (GATHER && xrow_ok[i]) src = perm[src];
        xrow_src[i] = src;
    }
    const int xchunk = tid & 3;

    uint32_t wreg[4];
    uint32_t xreg[2][4];
    auto load_global = [&](int kt) {
        const int w0 = kt * (kBK / 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) wreg[i] = 0x55555555u;
        if (wrow < pb.N) {
            if (waligned && w0 + 3 < W16) {
                const uint4 v = *reinterpret_cast<const uint4*>(wsrc + w0);
                wreg[0] = v.x; wreg[1] = v.y; wreg[2] = v.z; wreg[3] = v.w;
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (w0 + i < W16) wreg[i] = wsrc[w0 + i];
            }
        }
        const int k = kt * kBK + xchunk * 16;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            uint32_t d[4] = {0u, 0u, 0u, 0u};
            if (xrow_ok[i] && k < pb.K) {
                const uint4 v =
                    *reinterpret_cast<const uint4*>(q + (int64_t)xrow_src[i] * pb.K + k);
                d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
            }
            transpose16(d, xreg[i]);
        }
    };
    auto store_lds = [&](int buf) {
        *reinterpret_cast<uint4*>(wlds[buf] + tid * 4) =
            make_uint4(wreg[0], wreg[1], wreg[2], wreg[3]);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int ml = (tid >> 2) + 64 * i;
            *reinterpret_cast<uint4*>(xlds[buf] + ml * kXStride + xchunk * 16) =
                make_uint4(xreg[i][0], xreg[i][1], xreg[i][2], xreg[i][3]);
        }
    };

    v4i acc[8][4];
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = v4i{0, 0, 0, 0};

    load_global(0);
    store_lds(0);
    __syncthreads();

    const int g = lane >> 4;     // k group of 16
    const int li = lane & 15;    // row / column within a 16 x 16 tile
    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < KT) load_global(kt + 1);
        v4i bx[4];
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
            const int ml = wm * 64 + mb * 16 + li;
            const uint4 v = *reinterpret_cast<const uint4*>(xlds[cur] + ml * kXStride + g * 16);
            bx[mb] = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
        }
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) {
            const int nl = wn * 128 + nb * 16 + li;
            const uint32_t p = wlds[cur][nl * 4 + g];
            uint32_t wv[4];
            unpack_word(p, wv);
            const v4i aw = v4i{(int)wv[0], (int)wv[1], (int)wv[2], (int)wv[3]};
#pragma unroll
            for (int mb = 0; mb < 4; ++mb)
                acc[nb][mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aw, bx[mb], acc[nb][mb], 0, 0, 0);
        }
        if (kt + 1 < KT) store_lds(cur ^ 1);
        __syncthreads();
    }

    // epilogue: lane holds n = n_base + 4*g + r for token m = m_base + li
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
        const int ml = m0 + wm * 64 + mb * 16 + li;
        if (ml >= seg_rows) continue;
        const int64_t orow = (int64_t)(seg_begin + ml);
        const int arow = GATHER ? perm[seg_begin + ml] : (int)orow;
        const float comb = __fmul_rn(act_scale[arow], pb.ws);
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) {
            const int nbase = n0 + wn * 128 + nb * 16 + 4 * g;
            const v4i a = acc[nb][mb];
            const int av[4] = {a.x, a.y, a.z, a.w};
            if (ACC_OUT) {
                if (nbase + 3 < pb.N && (pb.N & 3) == 0) {
                    *reinterpret_cast<int4*>(acc_out + orow * pb.N + nbase) =
                        make_int4(av[0], av[1], av[2], av[3]);
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (nbase + r < pb.N) acc_out[orow * pb.N + nbase + r] = av[r];
                }
            }
            if (y) {
                float o[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int n = min(nbase + r, pb.N - 1);
                    float v = dequant(av[r], comb, pb.mag, pb.bias, n);
                    if (SQRELU) {
                        v = v > 0.0f ? v : 0.0f;
                        v = __fmul_rn(v, v);
                    }
                    o[r] = v;
                }
                if (nbase + 3 < pb.N && (pb.N & 3) == 0) {
                    if constexpr (YDT == NSOSX_F32) {
                        *reinterpret_cast<float4*>(static_cast<float*>(y) + orow * pb.N + nbase) =
                            make_float4(o[0], o[1], o[2], o[3]);
                    } else {
                        const uint32_t lo = f32_to_bf16(o[0]) | ((uint32_t)f32_to_bf16(o[1]) << 16);
                        const uint32_t hi = f32_to_bf16(o[2]) | ((uint32_t)f32_to_bf16(o[3]) << 16);
                        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(y) + orow * pb.N + nbase) =
                            make_uint2(lo, hi);
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (nbase + r < pb.N) store_act<YDT>(y, orow * pb.N + nbase + r, o[r]);
                }
            }
        }
    }
}

constexpr int kGemmSmem = 2 * kBN * 16 + 2 * kBM * kXStride;

// ===========================================================================
// Large-tile int8 MFMA GEMM (M > 128).  Block tile 256 (n) x 256 (m), eight
// waves in 4 (n) x 2 (m), each wave 64 n x 128 m = 2 x 4 tiles of
// v_mfma_i32_32x32x32_i8 (128 accumulators per lane, 8 independent chains:
// the 32x32 shape keeps the matrix pipe full where 16x16x64 with as many
// chains does not).  A stage covers 128 of K (four MFMA k steps, 32 MFMAs
// per wave); two LDS stages alternate, the next stage's global loads in
// flight across the current one's MFMAs.  Weights stay 2-bit in LDS (32
// bytes per row per stage) and are expanded in registers right before the
// MFMAs; the 8-byte pairs of a row are XOR-swizzled by (row / 8) % 4 so the
// 64 lanes of a fragment read hit 64 distinct banks.  Activation rows are
// byte-transposed into the unpack order on their way to LDS (row stride 144
// bytes: conflict-free 16-byte fragment reads).
// MFMA 32x32x32 lane layout: A row i = lane % 32 and B column j = lane % 32
// with k group lane / 32 (16 consecutive k each); accumulator r of a lane is
// C[i = 8 (r / 4) + 4 (lane / 32) + r % 4][j = lane % 32].
// ===========================================================================
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kBN2 = 256, kBM2 = 256, kBK2 = 128;
constexpr int kXS2 = 144;
constexpr int kW2Bytes = kBN2 * 32;
constexpr int kX2Bytes = kBM2 * kXS2;
constexpr int kGemm2Smem = 2 * (kW2Bytes + kX2Bytes);
constexpr int kGemm2Threads = 512;

template <int YDT, bool ACC_OUT, bool GATHER, bool SQRELU>
__device__ __forceinline__ void gemm2_tile(const GemmProblem& pb, const int8_t* __restrict__ q,
                                           const float* __restrict__ act_scale,
                                           const int32_t* __restrict__ perm, int seg_begin,
                                           int seg_rows, int n0, int m0, void* y,
                                           int32_t* acc_out, char* smem) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wn = wave & 3, wm = wave >> 2;
    const int W16 = pb.K >> 4;
    const int KT = (pb.K + kBK2 - 1) / kBK2;
    const bool waligned = (W16 & 3) == 0;

    // global -> register staging: half of a weight row's 32 bytes, four 16-byte
    // activation chunks
    const int wrow_l = tid >> 1, whalf = tid & 1;
    const int wrow = n0 + wrow_l;
    const uint32_t* wsrc = pb.packed + (int64_t)wrow * W16 + whalf * 4;
    const int xchunk = tid & 7;
    int xsrc[4];
    bool xok[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + (tid >> 3) + 64 * i;
        xok[i] = m < seg_rows;
        int src = seg_begin + m;
        if (GATHER && xok[i]) src = perm[src];
        xsrc[i] = src;
    }
    uint4 wreg;
    uint4 xraw[4];
    auto load_global = [&](int kt) {
        const int w0 = kt * (kBK2 / 16) + whalf * 4;
        wreg = make_uint4(0x55555555u, 0x55555555u, 0x55555555u, 0x55555555u);
        if (wrow < pb.N) {
            const uint32_t* src = wsrc + kt * (kBK2 / 16);
            if (waligned && w0 + 3 < W16) {
                wreg = *reinterpret_cast<const uint4*>(src);
            } else {
                if (w0 + 0 < W16) wreg.x = src[0];
                if (w0 + 1 < W16) wreg.y = src[1];
                if (w0 + 2 < W16) wreg.z = src[2];
                if (w0 + 3 < W16) wreg.w = src[3];
            }
        }
        const int k = kt * kBK2 + xchunk * 16;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            xraw[i] = make_uint4(0u, 0u, 0u, 0u);
            if (xok[i] && k < pb.K)
                xraw[i] = *reinterpret_cast<const uint4*>(q + (int64_t)xsrc[i] * pb.K + k);
        }
    };
    auto store_lds = [&](int buf) {
        char* wl = smem + buf * (kW2Bytes + kX2Bytes);
        char* xl = wl + kW2Bytes;
        // pairs 2h, 2h+1 of the row go to pair slots (2h)^f, (2h+1)^f
        const int f = (wrow_l >> 3) & 3;
        uint4 v = wreg;
        if (f & 1) v = make_uint4(v.z, v.w, v.x, v.y);
        *reinterpret_cast<uint4*>(wl + wrow_l * 32 + ((whalf ^ (f >> 1)) * 16)) = v;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t d[4] = {xraw[i].x, xraw[i].y, xraw[i].z, xraw[i].w};
            uint32_t e[4];
            transpose16(d, e);
            const int ml = (tid >> 3) + 64 * i;
            *reinterpret_cast<uint4*>(xl + ml * kXS2 + xchunk * 16) = make_uint4(e[0], e[1], e[2], e[3]);
        }
    };

    v16i acc[2][4];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = v16i{};

    load_global(0);
    store_lds(0);
    __syncthreads();

    const int g = lane >> 5;     // k group of 16
    const int li = lane & 31;    // row (A) / column (B) within a 32 x 32 tile
    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < KT) load_global(kt + 1);
        const uint32_t* wl = reinterpret_cast<const uint32_t*>(smem + cur * (kW2Bytes + kX2Bytes));
        const char* xl = smem + cur * (kW2Bytes + kX2Bytes) + kW2Bytes;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            v4i aw[2];
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
                const int nl = wn * 64 + nb * 32 + li;
                const int w = (ks * 2 + g) ^ (((nl >> 3) & 3) << 1);
                uint32_t wv[4];
                unpack_word(wl[nl * 8 + w], wv);
                aw[nb] = v4i{(int)wv[0], (int)wv[1], (int)wv[2], (int)wv[3]};
            }
            v4i bx[4];
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) {
                const int ml = wm * 128 + mb * 32 + li;
                const uint4 v = *reinterpret_cast<const uint4*>(xl + ml * kXS2 + ks * 32 + g * 16);
                bx[mb] = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
            }
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                for (int mb = 0; mb < 4; ++mb)
                    acc[nb][mb] =
                        __builtin_amdgcn_mfma_i32_32x32x32_i8(aw[nb], bx[mb], acc[nb][mb], 0, 0, 0);
        }
        if (kt + 1 < KT) store_lds(cur ^ 1);
        __syncthreads();
    }

    // epilogue: lane holds token m = m_base + li and, for q4 = 0..3, the four
    // consecutive outputs n = n_base + 8 q4 + 4 g + 0..3
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
        const int ml = m0 + wm * 128 + mb * 32 + li;
        if (ml >= seg_rows) continue;
        const int64_t orow = (int64_t)(seg_begin + ml);
        const int arow = GATHER ? perm[seg_begin + ml] : (int)orow;
        const float comb = __fmul_rn(act_scale[arow], pb.ws);
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const int nbase = n0 + wn * 64 + nb * 32 + 8 * q4 + 4 * g;
                const v16i& a = acc[nb][mb];
                const int av[4] = {a[4 * q4], a[4 * q4 + 1], a[4 * q4 + 2], a[4 * q4 + 3]};
                const bool full = nbase + 3 < pb.N && (pb.N & 3) == 0;
                if (ACC_OUT) {
                    if (full) {
                        *reinterpret_cast<int4*>(acc_out + orow * pb.N + nbase) =
                            make_int4(av[0], av[1], av[2], av[3]);
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (nbase + r < pb.N) acc_out[orow * pb.N + nbase + r] = av[r];
                    }
                }
                if (y) {
                    float o[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int n = min(nbase + r, pb.N - 1);
                        float v = dequant(av[r], comb, pb.mag, pb.bias, n);
                        if (SQRELU) {
                            v = v > 0.0f ? v : 0.0f;
                            v = __fmul_rn(v, v);
                        }
                        o[r] = v;
                    }
                    if (full) {
                        if constexpr (YDT == NSOSX_F32) {
                            *reinterpret_cast<float4*>(static_cast<float*>(y) + orow * pb.N + nbase) =
                                make_float4(o[0], o[1], o[2], o[3]);
                        } else {
                            const uint32_t lo = f32_to_bf16(o[0]) | ((uint32_t)f32_to_bf16(o[1]) << 16);
                            const uint32_t hi = f32_to_bf16(o[2]) | ((uint32_t)f32_to_bf16(o[3]) << 16);
                            *reinterpret_cast<uint2*>(static_cast<uint16_t*>(y) + orow * pb.N + nbase) =
                                make_uint2(lo, hi);
                        }
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (nbase + r < pb.N) store_act<YDT>(y, orow * pb.N + nbase + r, o[r]);
                    }
                }
            }
        }
    }
}

// ===========================================================================
// LDS-staged int8 MFMA GEMM (M > 128, K % 128 == 0).  Block tile 256 (n)
// x 128 (m), four waves each owning 64 n x 128 m = 2 x 4 tiles of
// v_mfma_i32_32x32x32_i8 (128 accumulators, 8 independent chains).  Each stage
// is fetched into registers with 16-byte loads two stages ahead and written
// into a 3-stage ring of 128-deep K stages (24 KB each, 72 KB in all), so two
// workgroups share a CU and their barrier phases interleave.
// K mapping inside a stage: MFMA step ks, lane group g (lane / 32) takes the
// 16 k values of chunk 4 g + ks, so each lane's weights for the whole stage
// are one 16-byte packed word group (read once, decoded one word per step)
// and its activations one 16-byte chunk per step.  Bank spreading (64 banks
// of 4 bytes; a 16-byte read serves 16 lanes per clock), chosen through
// which global chunk each lane fetches:
//   weights     the two 16-byte halves of row r swap when (r / 8) is odd
//   activations 16-byte chunk c of row r sits in slot c ^ ((r / 2) % 8)
// Activation rows land in natural byte order; a reference-layout weight word is
// byte-transposed to match after decoding (the MFMA layout decodes into natural
// order directly).  Rows past N or M are fetched from a clamped, in-bounds row;
// their outputs are never stored.
// ===========================================================================
constexpr int kG3BN = 256, kG3BM = 128, kG3BK = 128;
constexpr int kG3Stages = 3;
constexpr int kG3WBytes = kG3BN * 32;     // 8 KB
constexpr int kG3XBytes = kG3BM * 128;    // 16 KB
constexpr int kG3StageBytes = kG3WBytes + kG3XBytes;
constexpr int kGemm3Smem = kG3Stages * kG3StageBytes;
constexpr int kGemm3Threads = 256;

// 16-byte load of a stage through a global-memory pointer (a flat load would also
// count against the LDS wait counter the stage loop drains before its barrier).
__device__ __forceinline__ uint4 load_stage16(const char* p) {
    const u32x4 v = *(global_u32x4*)(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// MFMA layout word -> the 16 int8 operand bytes of codes k = 0..15 in natural
// order, each 64 x its ternary value: code k is a two's-complement 2-bit field at
// bits 8 (k % 4) + 6 - 2 (k / 4), so dword s (codes 4s .. 4s+3) is the word
// shifted left by 2s with all but the top two bits of every byte cleared.  The
// accumulators come out 64 x the true sums (exact in int32 for K < 2^18 / 127).
constexpr int kMfmaLayoutMaxK = 2147483647 / (64 * 127);  // 64 * 127 * K fits int32
__device__ __forceinline__ v4i unpack_word_mfma(uint32_t w) {
    return v4i{(int)(w & 0xC0C0C0C0u), (int)((w << 2) & 0xC0C0C0C0u), (int)((w << 4) & 0xC0C0C0C0u),
               (int)((w << 6) & 0xC0C0C0C0u)};
}

// One 128-deep K stage of the 256 x 128 block from LDS stage `st`: each lane
// reads its two 16-byte weight word groups once, then per MFMA step ks decodes
// one word per n-tile and reads one 16-byte activation chunk per m-tile.
template <bool SWZ, int MB>
__device__ __forceinline__ void gemm3_stage(const char* st, int wave, int lane, v16i (&acc)[2][4]) {
    const int g = lane >> 5;
    const int li = lane & 31;
    const char* xl = st + kG3WBytes;
    uint4 wq[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        const int nl = wave * 64 + nb * 32 + li;
        const int slot = g ^ ((nl >> 3) & 1);
        wq[nb] = *reinterpret_cast<const uint4*>(st + nl * 32 + slot * 16);
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        v4i bx[4];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const int ml = mb * 32 + li;
            const int slot = (4 * g + ks) ^ ((ml >> 1) & 7);
            const uint4 v = *reinterpret_cast<const uint4*>(xl + ml * 128 + slot * 16);
            bx[mb] = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
        }
        v4i aw[2];
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            const uint32_t words[4] = {wq[nb].x, wq[nb].y, wq[nb].z, wq[nb].w};
            if constexpr (SWZ) {
                aw[nb] = unpack_word_mfma(words[ks]);       // 64 x the values, natural order
            } else {
                uint32_t wv[4], wt[4];
                unpack_word(words[ks], wv);
                transpose16(wv, wt);                        // unpack order -> natural order
                aw[nb] = v4i{(int)wt[0], (int)wt[1], (int)wt[2], (int)wt[3]};
            }
        }
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
                acc[nb][mb] =
                    __builtin_amdgcn_mfma_i32_32x32x32_i8(aw[nb], bx[mb], acc[nb][mb], 0, 0, 0);
    }
}

template <int YDT, bool ACC_OUT, bool GATHER, bool SQRELU>
__device__ __forceinline__ void gemm3_epilogue(const GemmProblem& pb,
                                               const float* __restrict__ act_scale,
                                               const int32_t* __restrict__ perm, int seg_begin,
                                               int seg_rows, int n0, int m0, void* y,
                                               int32_t* acc_out, const v16i (&acc)[2][4]) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = lane >> 5;
    const int li = lane & 31;
    // epilogue: lane holds token m = m_base + li and, for q4 = 0..3, the four
    // consecutive outputs n = n_base + 8 q4 + 4 g + 0..3.  A tile that lies
    // inside N (N % 4 == 0) stores 4 outputs per access at constant offsets from
    // one row pointer; edge tiles go element by element.
    const bool full_tile = n0 + kG3BN <= pb.N && (pb.N & 3) == 0;
    const int nw = n0 + wave * 64 + 4 * g;  // this lane's first output column
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
        const int ml = m0 + mb * 32 + li;
        if (ml >= seg_rows) continue;
        const int64_t orow = (int64_t)(seg_begin + ml);
        const int arow = GATHER ? perm[seg_begin + ml] : (int)orow;
        const float comb = __fmul_rn(act_scale[arow], pb.ws);
        if (full_tile) {
            int32_t* arow_out = ACC_OUT ? acc_out + orow * pb.N + nw : nullptr;
            char* yrow = y ? static_cast<char*>(y) + (orow * pb.N + nw) * (YDT == NSOSX_F32 ? 4 : 2)
                           : nullptr;
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    const int off = nb * 32 + 8 * q4;
                    const v16i& a = acc[nb][mb];
                    if (ACC_OUT)
                        *reinterpret_cast<int4*>(arow_out + off) =
                            make_int4(a[4 * q4], a[4 * q4 + 1], a[4 * q4 + 2], a[4 * q4 + 3]);
                    if (y) {
                        float o[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            float v = dequant(a[4 * q4 + r], comb, pb.mag, pb.bias, nw + off + r);
                            if (SQRELU) {
                                v = v > 0.0f ? v : 0.0f;
                                v = __fmul_rn(v, v);
                            }
                            o[r] = v;
                        }
                        if constexpr (YDT == NSOSX_F32) {
                            *reinterpret_cast<float4*>(yrow + off * 4) = make_float4(o[0], o[1], o[2], o[3]);
                        } else {
                            *reinterpret_cast<uint2*>(yrow + off * 2) =
                                make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]));
                        }
                    }
                }
            }
            continue;
        }
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const int nbase = nw + nb * 32 + 8 * q4;
                const v16i& a = acc[nb][mb];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int n = nbase + r;
                    if (n >= pb.N) continue;
                    if (ACC_OUT) acc_out[orow * pb.N + n] = a[4 * q4 + r];
                    if (y) {
                        float v = dequant(a[4 * q4 + r], comb, pb.mag, pb.bias, n);
                        if (SQRELU) {
                            v = v > 0.0f ? v : 0.0f;
                            v = __fmul_rn(v, v);
                        }
                        store_act<YDT>(y, orow * pb.N + n, v);
                    }
                }
            }
        }
    }
}

// bf16 epilogue of a tile that lies inside N (N % 8 == 0).  The accumulator
// layout scatters a store instruction over 32 rows at 8 bytes per lane; here
// each wave instead dequantizes its 64 n x 128 m block into a private 16 KB
// slice of the idle stage ring as 128 rows of 64 bf16 (128 bytes), then stores
// whole row segments: one instruction writes 8 rows, 16 bytes per lane, each
// row one aligned 128-byte line.  In a slice, 16-byte chunk c of row r sits in
// slot c ^ ((r / 2) % 8), so neither the 8-byte writes (32 rows, one chunk)
// nor the 16-byte reads (8 rows, 8 chunks) conflict on the 64 banks.
// Magnitude, bias and every output pointer must be 16-byte aligned.  MAG / BIAS
// are template arguments (the caller branches once on the pointers): as runtime
// conditions the compiler formed both results per element and selected one.
template <bool GATHER, bool SQRELU, bool MAG, bool BIAS>
__device__ __forceinline__ void gemm3_epilogue_rows(const GemmProblem& pb,
                                                    const float* __restrict__ act_scale,
                                                    const int32_t* __restrict__ perm, int seg_begin,
                                                    int seg_rows, int n0, int m0, uint16_t* y,
                                                    const v16i (&acc)[2][4], char* smem) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = lane >> 5;
    const int li = lane & 31;
    const int nw = n0 + wave * 64 + 4 * g;  // this lane's first output column
    float comb[4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
        const int ml = min(m0 + mb * 32 + li, seg_rows - 1);  // rows past the segment are never stored
        const int arow = GATHER ? perm[seg_begin + ml] : seg_begin + ml;
        comb[mb] = __fmul_rn(act_scale[arow], pb.ws);
    }
    __syncthreads();  // every wave is done reading the stage ring
    char* slice = smem + wave * (kG3BM * 128);
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            const int n = nw + nb * 32 + 8 * q4;
            const float4 mg = MAG ? *reinterpret_cast<const float4*>(pb.mag + n) : float4{};
            const float4 bs = BIAS ? *reinterpret_cast<const float4*>(pb.bias + n) : float4{};
            const float mv[4] = {mg.x, mg.y, mg.z, mg.w};
            const float bv[4] = {bs.x, bs.y, bs.z, bs.w};
            const int c = nb * 4 + q4;
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) {
                const v16i& a = acc[nb][mb];
                float o[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float v = __fmul_rn(static_cast<float>(a[4 * q4 + r]), comb[mb]);
                    if (MAG) v = __fmul_rn(v, mv[r]);
                    if (BIAS) v = __fadd_rn(v, bv[r]);
                    if (SQRELU) {
                        v = v > 0.0f ? v : 0.0f;
                        v = __fmul_rn(v, v);
                    }
                    o[r] = v;
                }
                const int row = mb * 32 + li;
                *reinterpret_cast<uint2*>(slice + row * 128 + g * 8 + ((c ^ ((row >> 1) & 7)) << 4)) =
                    make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]));
            }
        }
    // The wave reads back what its own lanes wrote: LDS operations of one wave
    // complete in order, and the wait keeps the compiler from hoisting the reads.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const int c = lane & 7;
    uint16_t* ycol = y + n0 + wave * 64 + c * 8;
#pragma unroll
    for (int i = 0; i < kG3BM / 8; ++i) {
        const int row = i * 8 + (lane >> 3);
        const uint4 v = *reinterpret_cast<const uint4*>(slice + row * 128 + ((c ^ ((row >> 1) & 7)) << 4));
        // non-temporal: the output is not read again by this launch, and streaming it past
        // the caches keeps the stage loads' weights and codes resident (in_proj +11 %)
        if (m0 + row < seg_rows)
            __builtin_nontemporal_store(u32x4{v.x, v.y, v.z, v.w},
                                        reinterpret_cast<u32x4*>(ycol + (int64_t)(seg_begin + m0 + row) * pb.N));
    }
}

// f32 epilogue of a tile that lies inside N (N % 4 == 0), staged like the bf16 one:
// a wave's 64 n x 128 m block is 32 KB of floats, so it goes out in two halves of
// 64 rows (mb 0-1, then 2-3) through the wave's 16 KB slice of the idle ring, each
// row 256 bytes (16 chunks of 16 bytes, chunk c of row r at slot c ^ (r % 16): the
// 16-byte writes of 16 rows and the reads of one row's 16 chunks are conflict-free).
// One store instruction then writes 4 rows as whole 256-byte segments.
template <bool GATHER, bool SQRELU, bool MAG, bool BIAS>
__device__ __forceinline__ void gemm3_epilogue_rows_f32(const GemmProblem& pb,
                                                        const float* __restrict__ act_scale,
                                                        const int32_t* __restrict__ perm,
                                                        int seg_begin, int seg_rows, int n0, int m0,
                                                        float* y, const v16i (&acc)[2][4],
                                                        char* smem) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = lane >> 5;
    const int li = lane & 31;
    const int nw = n0 + wave * 64 + 4 * g;  // this lane's first output column
    float comb[4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
        const int ml = min(m0 + mb * 32 + li, seg_rows - 1);  // rows past the segment are never stored
        const int arow = GATHER ? perm[seg_begin + ml] : seg_begin + ml;
        comb[mb] = __fmul_rn(act_scale[arow], pb.ws);
    }
    __syncthreads();  // every wave is done reading the stage ring
    char* slice = smem + wave * (kG3BM * 128);
    float* ycol = y + n0 + wave * 64 + (lane & 15) * 4;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const int c = nb * 8 + 2 * q4 + g;  // this lane's 16-byte chunk of the row
                const int n = nw + nb * 32 + 8 * q4;
                const float4 mg = MAG ? *reinterpret_cast<const float4*>(pb.mag + n) : float4{};
                const float4 bs = BIAS ? *reinterpret_cast<const float4*>(pb.bias + n) : float4{};
                const float mv[4] = {mg.x, mg.y, mg.z, mg.w};
                const float bv[4] = {bs.x, bs.y, bs.z, bs.w};
#pragma unroll
                for (int mh = 0; mh < 2; ++mh) {
                    const int mb = 2 * half + mh;
                    const v16i& a = acc[nb][mb];
                    float o[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float v = __fmul_rn(static_cast<float>(a[4 * q4 + r]), comb[mb]);
                        if (MAG) v = __fmul_rn(v, mv[r]);
                        if (BIAS) v = __fadd_rn(v, bv[r]);
                        if (SQRELU) {
                            v = v > 0.0f ? v : 0.0f;
                            v = __fmul_rn(v, v);
                        }
                        o[r] = v;
                    }
                    const int row = mh * 32 + li;
                    *reinterpret_cast<float4*>(slice + row * 256 + ((c ^ (row & 15)) << 4)) =
                        make_float4(o[0], o[1], o[2], o[3]);
                }
            }
        // the wave reads back what its own lanes wrote (LDS operations of one wave
        // complete in order; the wait keeps the compiler from hoisting the reads)
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const int c = lane & 15;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int row = i * 4 + (lane >> 4);
            const float4 v = *reinterpret_cast<const float4*>(slice + row * 256 + ((c ^ (row & 15)) << 4));
            const int m = m0 + half * 64 + row;
            if (m < seg_rows)  // non-temporal, as the bf16 epilogue
                __builtin_nontemporal_store(
                    u32x4{__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)},
                    reinterpret_cast<u32x4*>(ycol + (int64_t)(seg_begin + m) * pb.N));
        }
        // the next half overwrites the slice: its writes follow these reads in order
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
}

// MB: 32-row blocks of the tile that hold rows (a partial last tile of an expert's
// segment skips the loads and MFMAs of its empty blocks; their accumulators stay zero
// and their rows are never stored).
template <int YDT, bool ACC_OUT, bool GATHER, bool SQRELU, bool SWZ = false, int MB = 4>
__device__ __forceinline__ void gemm3_tile(const GemmProblem& pb, const int8_t* __restrict__ q,
                                           const float* __restrict__ act_scale,
                                           const int32_t* __restrict__ perm, int seg_begin,
                                           int seg_rows, int n0, int m0, void* y,
                                           int32_t* acc_out, char* smem) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;        // wave = 64-row slice of n
    const int W16 = pb.K >> 4;
    const int KT = pb.K / kG3BK;

    // Stage sources.  Weights: wave-load j (0, 1) of a wave fills LDS rows
    // 64 wave + 32 j .. +31, lane -> row + lane / 2, slot lane % 2.
    const char* wsrc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int r = 64 * wave + 32 * j + (lane >> 1);
        const int half = (lane & 1) ^ ((r >> 3) & 1);
        const int row = min(n0 + r, pb.N - 1);
        wsrc[j] = reinterpret_cast<const char*>(pb.packed + (int64_t)row * W16) + half * 16;
    }
    // Activations: wave-load i (0..3) of a wave fills LDS rows 32 i + 8 wave .. +7,
    // lane -> row + lane / 8, slot lane % 8.
    const char* xsrc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = 32 * i + 8 * wave + (lane >> 3);
        const int c = (lane & 7) ^ ((r >> 1) & 7);
        const int m = min(m0 + r, seg_rows - 1);
        const int src = GATHER ? perm[seg_begin + m] : seg_begin + m;
        xsrc[i] = reinterpret_cast<const char*>(q + (int64_t)src * pb.K) + c * 16;
    }
    // Stage kt is fetched into registers at iteration kt - 2 (16-byte loads: 2 of
    // weights, MB of activations per lane) and written to its LDS slot at kt - 1;
    // the slot it overwrites was last read at kt - 3, before the barrier of kt - 2.
    // (global_load_lds straight into LDS was measured slower: its LDS writes stall
    // the MFMA stream even when the data is already in L2.)
    uint4 rw0, rw1, rx0, rx1, rx2, rx3;
    auto fetch = [&](int kt) {
        rw0 = load_stage16(wsrc[0] + kt * 32);
        rw1 = load_stage16(wsrc[1] + kt * 32);
        rx0 = load_stage16(xsrc[0] + kt * 128);
        if (MB > 1) rx1 = load_stage16(xsrc[1] + kt * 128);
        if (MB > 2) rx2 = load_stage16(xsrc[2] + kt * 128);
        if (MB > 3) rx3 = load_stage16(xsrc[3] + kt * 128);
    };
    auto put = [&](int kt) {
        char* st = smem + (kt % kG3Stages) * kG3StageBytes + lane * 16;
        *reinterpret_cast<uint4*>(st + (64 * wave) * 32) = rw0;
        *reinterpret_cast<uint4*>(st + (64 * wave + 32) * 32) = rw1;
        char* sx = st + kG3WBytes + (8 * wave) * 128;
        *reinterpret_cast<uint4*>(sx) = rx0;
        if (MB > 1) *reinterpret_cast<uint4*>(sx + 32 * 128) = rx1;
        if (MB > 2) *reinterpret_cast<uint4*>(sx + 64 * 128) = rx2;
        if (MB > 3) *reinterpret_cast<uint4*>(sx + 96 * 128) = rx3;
    };

    v16i acc[2][4];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = v16i{};

    fetch(0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    put(0);
    if (KT > 1) fetch(1);
    for (int kt = 0; kt < KT; ++kt) {
        if (kt + 1 < KT) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // stage kt + 1 is in registers
            put(kt + 1);
            if (kt + 2 < KT) fetch(kt + 2);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        gemm3_stage<SWZ, MB>(smem + (kt % kG3Stages) * kG3StageBytes, wave, lane, acc);
    }
    if constexpr (SWZ) {
        // MFMA-layout operands carry 64 x the ternary values (unpack_word_mfma)
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 4; ++b)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[a][b][e] >>= 6;
    }

    if constexpr (YDT == NSOSX_BF16 && !ACC_OUT) {
        if (y && n0 + kG3BN <= pb.N && (pb.N & 7) == 0 &&
            ((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(pb.mag) |
              reinterpret_cast<uintptr_t>(pb.bias)) & 15) == 0) {
            uint16_t* yb = static_cast<uint16_t*>(y);
#define NSOSX_EPI(MG, BS)                                                                       \
    gemm3_epilogue_rows<GATHER, SQRELU, MG, BS>(pb, act_scale, perm, seg_begin, seg_rows, n0, m0, \
                                                yb, acc, smem)
            if (pb.mag) {
                if (pb.bias) NSOSX_EPI(true, true); else NSOSX_EPI(true, false);
            } else {
                if (pb.bias) NSOSX_EPI(false, true); else NSOSX_EPI(false, false);
            }
#undef NSOSX_EPI
            return;
        }
    }
    if constexpr (YDT == NSOSX_F32 && !ACC_OUT) {
        if (y && n0 + kG3BN <= pb.N && (pb.N & 3) == 0 &&
            ((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(pb.mag) |
              reinterpret_cast<uintptr_t>(pb.bias)) & 15) == 0) {
            float* yf = static_cast<float*>(y);
#define NSOSX_EPI(MG, BS)                                                                 \
    gemm3_epilogue_rows_f32<GATHER, SQRELU, MG, BS>(pb, act_scale, perm, seg_begin, seg_rows, n0, \
                                                    m0, yf, acc, smem)
            if (pb.mag) {
                if (pb.bias) NSOSX_EPI(true, true); else NSOSX_EPI(true, false);
            } else {
                if (pb.bias) NSOSX_EPI(false, true); else NSOSX_EPI(false, false);
            }
#undef NSOSX_EPI
            return;
        }
    }
    gemm3_epilogue<YDT, ACC_OUT, GATHER, SQRELU>(pb, act_scale, perm, seg_begin, seg_rows, n0, m0,
                                                 y, acc_out, acc);
}

// Linear workgroup id -> (n tile, m tile).  Consecutive ids go round-robin to
// the 8 XCDs; this map hands each XCD a contiguous run of tiles, n fastest,
// so the workgroups of one XCD share activation rows in their own L2.
__device__ __forceinline__ void xcd_tile(int L, int ntn, int ntm, int& nt, int& mt) {
    const int total = ntn * ntm;
    const int per = total / 8;
    int t = L;
    if (L < per * 8) t = (L % 8) * per + L / 8;
    nt = t % ntn;
    mt = t / ntn;
}

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

// Tile L of a grouped launch over the experts' real row tiles: every expert's full
// 128-row tiles first (XCD-swizzled, n fastest), then each expert's partial last
// tile, so that the partial tiles, cheaper by their skipped empty 32-row blocks,
// make up the last round of a launch that does not divide into whole rounds.
__device__ __forceinline__ bool grouped_tile(const int32_t* __restrict__ offsets, int experts,
                                             int ntn, int L, int& nt, int& e, int& seg_begin,
                                             int& seg_rows, int& m0) {
    int full = 0;
    for (int j = 0; j < experts; ++j) full += max(offsets[j + 1] - offsets[j], 0) / kG3BM;
    if (L < ntn * full) {
        int rest;
        xcd_tile(L, ntn, full, nt, rest);
        int base = 0;
        for (int j = 0; j < experts; ++j) {
            const int b = offsets[j];
            const int f = max(offsets[j + 1] - b, 0) / kG3BM;
            if (rest < base + f) {
                e = j; seg_begin = b; seg_rows = offsets[j + 1] - b; m0 = (rest - base) * kG3BM;
                return true;
            }
            base += f;
        }
        return false;
    }
    const int idx = L - ntn * full;
    nt = idx % ntn;
    int p = idx / ntn;
    for (int j = 0; j < experts; ++j) {
        const int b = offsets[j];
        const int r = max(offsets[j + 1] - b, 0);
        if (r % kG3BM == 0) continue;
        if (p == 0) {
            e = j; seg_begin = b; seg_rows = r; m0 = (r / kG3BM) * kG3BM;
            return true;
        }
        --p;
    }
    return false;
}

// gemm3_tile with the 32-row blocks that hold rows of the segment
template <int YDT, bool GATHER, bool SQRELU, bool SWZ>
__device__ __forceinline__ void gemm3_tile_rows(const GemmProblem& pb, const int8_t* __restrict__ q,
                                                const float* __restrict__ act_scale,
                                                const int32_t* __restrict__ perm, int seg_begin,
                                                int seg_rows, int n0, int m0, void* y, char* smem) {
    const int rows = seg_rows - m0;
    if (rows > 96)
        gemm3_tile<YDT, false, GATHER, SQRELU, SWZ, 4>(pb, q, act_scale, perm, seg_begin, seg_rows,
                                                        n0, m0, y, nullptr, smem);
    else if (rows > 64)
        gemm3_tile<YDT, false, GATHER, SQRELU, SWZ, 3>(pb, q, act_scale, perm, seg_begin, seg_rows,
                                                        n0, m0, y, nullptr, smem);
    else if (rows > 32)
        gemm3_tile<YDT, false, GATHER, SQRELU, SWZ, 2>(pb, q, act_scale, perm, seg_begin, seg_rows,
                                                        n0, m0, y, nullptr, smem);
    else
        gemm3_tile<YDT, false, GATHER, SQRELU, SWZ, 1>(pb, q, act_scale, perm, seg_begin, seg_rows,
                                                        n0, m0, y, nullptr, smem);
}

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

// ===========================================================================
// Skinny GEMM for decode batches (2 <= M <= 32 token rows) on
// v_mfma_i32_16x16x64_i8.  A tile is 16 weight rows x 16 tokens (one or two m
// tiles); MFMA step s covers k = 64 s .. 64 s + 63, and lane (g, li) =
// (lane / 16, lane % 16) feeds row li of the tile with k group g of the step:
// one packed word (16 codes) per step, decoded in registers and used in unpack
// order.  The activation fragments (token li, the same 16 k) are byte-transposed
// into that order once per workgroup (16 bytes per lane per step and m tile,
// M_pad x K bytes of LDS); the first m tile's stay in registers up to K = 2048.
// A wave streams its tiles with the next tile's loads in flight; the dot costs
// one decode per word whatever M is, so the kernel stays HBM-bound where the
// VALU GEMV's per-row dot products do not.  Needs K in {1024, 2048, 4096} and
// ceil(M / 16) * K <= 4096.
// MFMA 16x16x64 lane layout: A row = lane % 16 and B column = lane % 16, k group
// lane / 16 (16 consecutive k); accumulator r is C[4 (lane / 16) + r][lane % 16].
// ===========================================================================
constexpr int kSkMaxLds = 64 * 1024;
constexpr size_t kGroupedSkinnyLds = 2 * 2048 * 16;  // one m tile at K <= 2048

// K = 256 * LT with LT (16-byte loads per lane per tile) in {4, 8, 16}; the
// outputs are addressed with 32-bit byte offsets below the 2^31 drop offset
static bool skinny_ok(int M, int K, int N) {
    const int mt = (M + 15) / 16;
    return M >= 2 && M <= 32 && (K == 1024 || K == 2048 || K == 4096) &&
           (int64_t)mt * K * 16 <= kSkMaxLds && (int64_t)M * N * 4 < ((int64_t)1 << 31);
}

// The steady state is straight-line code (the tile loop's back edge is its only
// branch), so the compiler keeps exact counts of the loads in flight: loads
// past the last tile are clamped into the matrix, and stores of rows past N or
// tokens past M go to an offset past the output's buffer extent, where the
// hardware drops them.
typedef uint32_t v2u __attribute__((ext_vector_type(2)));

// ML: the weights are in the MFMA layout (nsosx_pack_mfma_layout): each word decodes by
// shift and mask into natural k order (64 x the values, unpack_word_mfma), so the
// activation fragments stay in natural order and the sums are shifted back by 6.
template <int MT, int LT, int YDT, bool ACC_OUT, bool SQRELU, bool VEC4, bool ML = false>
__device__ __forceinline__ void skinny_body(const GemvProblem& pb, const int8_t* __restrict__ q,
                                            const float* __restrict__ act_scale, int M, void* y,
                                            int32_t* acc_out, int wave_id, int num_waves,
                                            char* lds) {
    constexpr int Q = 4 * LT;                       // words per lane per tile (MFMA steps)
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int g = lane >> 4, li = lane & 15;
    const int W16 = pb.K >> 4;
    // activation fragments: fragment (s, mt) of lane l at ((s * MT + mt) * 64 + l) * 16;
    // step s covers k = 64 s .. 64 s + 63, k group g its 16 k from 64 s + 16 g
    constexpr int nfrag = Q * MT * 64;
    for (int f = tid; f < nfrag; f += blockDim.x) {
        const int l = f & 63;
        const int smt = f >> 6;
        const int mt = smt % MT, st = smt / MT;
        const int m = mt * 16 + (l & 15);
        const int k0 = 16 * (4 * st + (l >> 4));
        uint32_t d[4] = {0u, 0u, 0u, 0u};
        if (m < M) {
            const uint4 v = *reinterpret_cast<const uint4*>(q + (int64_t)m * pb.K + k0);
            d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
        }
        uint32_t e[4] = {d[0], d[1], d[2], d[3]};
        if constexpr (!ML) transpose16(d, e);
        *reinterpret_cast<uint4*>(lds + f * 16) = make_uint4(e[0], e[1], e[2], e[3]);
    }
    __syncthreads();
    const int tiles = (pb.N + 15) >> 4;
    if (wave_id >= tiles) return;
    const int my_tiles = (tiles - 1 - wave_id) / num_waves + 1;
    // A tile's 16 rows are one contiguous block of 16 * K / 4 bytes.  The wave
    // reads it in LT loads of 1 KB (lane l: bytes 1024 j + 16 l), so every load
    // instruction covers eight whole 128-byte lines, and passes it through its own
    // LDS slice: 16-byte chunk c of row r sits at chunk c ^ (r % 16) of the row
    // (conflict-free both ways).  Read j of lane (g, li) is row li's 64 bytes
    // 64 j + 16 g (words 16 j + 4 g .. +3), i.e. k group u of steps 4 j + g; a
    // 4 x 4 transpose across the four 16-lane rows (v_permlane32_swap, then
    // v_permlane16_swap) turns that into k group g of steps 4 j + u.
    constexpr int RB = 64 * LT;                     // bytes per weight row
    char* stage = lds + MT * pb.K * 16 + (tid >> 6) * 16 * RB;
    const int64_t last_word = (int64_t)pb.N * W16 - 4;
    auto tile_src = [&](int ti) {
        const int tile = wave_id + min(ti, my_tiles - 1) * num_waves;
        return (int64_t)tile * 16 * W16 + 4 * lane;
    };
    auto load_piece = [&](int64_t base, int j) {
        return load_stream16(pb.packed + min(base + 256 * j, last_word));
    };
    constexpr uint32_t ES = YDT == NSOSX_F32 ? 4 : 2;
    const __amdgpu_buffer_rsrc_t ry =
        make_rsrc(y, y ? static_cast<uint32_t>(M * pb.N) * ES : 0u);
    const __amdgpu_buffer_rsrc_t racc =
        make_rsrc(acc_out, ACC_OUT ? static_cast<uint32_t>(M * pb.N) * 4u : 0u);
    float comb[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
        comb[mt] = __fmul_rn(act_scale[min(mt * 16 + li, M - 1)], pb.ws);

    // The affine terms of a tile's four output columns load with its weights (a null
    // magnitude or bias reads through an empty resource, which returns zeros), so the
    // epilogue waits on nothing the ring's loads do not already bring.
    const bool has_mag = pb.mag != nullptr, has_bias = pb.bias != nullptr;
    const __amdgpu_buffer_rsrc_t rmag = make_rsrc(pb.mag, has_mag ? pb.N * 4u : 0u);
    const __amdgpu_buffer_rsrc_t rbias = make_rsrc(pb.bias, has_bias ? pb.N * 4u : 0u);
    auto tile_n0 = [&](int ti) { return (wave_id + ti * num_waves) * 16 + 4 * g; };
    auto load_affine = [&](int ti, float (&mg)[4], float (&bs)[4]) {
        const uint32_t off = static_cast<uint32_t>(tile_n0(min(ti, my_tiles - 1))) * 4u;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            mg[r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rmag, off + 4 * r, 0, 0));
            bs[r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rbias, off + 4 * r, 0, 0));
        }
    };

    uint4 ring[LT];
    float mg_cur[4], bs_cur[4];
    {
        const int64_t b0 = tile_src(0);
#pragma unroll
        for (int j = 0; j < LT; ++j) ring[j] = load_piece(b0, j);
        load_affine(0, mg_cur, bs_cur);
    }
    const char* frag = lds + lane * 16;
    // the first m tile's fragments up to K = 2048 (512 bytes per lane) stay in
    // registers for the whole stream; the rest are re-read from LDS per tile
    constexpr bool kHold = LT <= 8;
    uint4 held[kHold ? 4 * LT : 1];
    if constexpr (kHold) {
#pragma unroll
        for (int st = 0; st < 4 * LT; ++st)
            held[st] = *reinterpret_cast<const uint4*>(frag + st * MT * 1024);
    }
    // Tiles go in batches of kSkBatch whose outputs are stored together after the
    // batch.  On this architecture a wait for loads issued while a store is in flight
    // waits for the store as well (loads and stores share one counter and may complete
    // out of order), so a store per tile would expose a store round trip at every
    // tile's wait for its weights; per batch it is one in kSkBatch.  The batch is
    // unrolled (straight-line, exact wait counts); tiles past the wave's last compute on
    // clamped loads and store nothing.
    constexpr int kSkBatch = 2;
    for (int t0 = 0; t0 < my_tiles; t0 += kSkBatch) {
        float vb[kSkBatch][MT][4];
        int ab[kSkBatch][MT][4];
#pragma unroll
        for (int u = 0; u < kSkBatch; ++u) {
            const int ti = t0 + u;
            // this tile to the wave's LDS slice (in order with the reads below), then
            // the next tile's loads into the ring
#pragma unroll
            for (int j = 0; j < LT; ++j) {
                const int b = 1024 * j + 16 * lane;
                const int r = b / RB, c = (b % RB) >> 4;
                *reinterpret_cast<uint4*>(stage + r * RB + ((c ^ (r & 15)) << 4)) = ring[j];
            }
            float mg_nxt[4], bs_nxt[4];
            {
                const int64_t nb0 = tile_src(ti + 1);
#pragma unroll
                for (int j = 0; j < LT; ++j) ring[j] = load_piece(nb0, j);
                load_affine(ti + 1, mg_nxt, bs_nxt);
            }
            v4i acc[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[mt] = v4i{0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < LT; ++j) {
                const uint4 w = *reinterpret_cast<const uint4*>(
                    stage + li * RB + (((4 * j + g) ^ li) << 4));
                // 4 x 4 transpose (16-lane row g, slot u) -> (row u, slot g)
                const auto p02 = __builtin_amdgcn_permlane32_swap(w.x, w.z, false, false);
                const auto p13 = __builtin_amdgcn_permlane32_swap(w.y, w.w, false, false);
                const auto p01 = __builtin_amdgcn_permlane16_swap(p02[0], p13[0], false, false);
                const auto p23 = __builtin_amdgcn_permlane16_swap(p02[1], p13[1], false, false);
                const uint32_t words[4] = {p01[0], p01[1], p23[0], p23[1]};
#pragma unroll
                for (int uu = 0; uu < 4; ++uu) {
                    v4i aw;
                    if constexpr (ML) {
                        aw = unpack_word_mfma(words[uu]);
                    } else {
                        uint32_t wv[4];
                        unpack_word(words[uu], wv);
                        aw = v4i{(int)wv[0], (int)wv[1], (int)wv[2], (int)wv[3]};
                    }
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        const uint4 v =
                            kHold && mt == 0
                                ? held[(4 * j + uu) % (kHold ? 4 * LT : 1)]
                                : *reinterpret_cast<const uint4*>(frag + ((4 * j + uu) * MT + mt) * 1024);
                        acc[mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                            aw, v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w}, acc[mt], 0, 0, 0);
                    }
                }
            }
            // lane holds outputs n = tile * 16 + 4 g + r of token mt * 16 + li
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                constexpr int sh = ML ? 6 : 0;
                const int av[4] = {acc[mt].x >> sh, acc[mt].y >> sh, acc[mt].z >> sh, acc[mt].w >> sh};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    // the reference's affine: multiply, then add, each rounded
                    float v = __fmul_rn(static_cast<float>(av[r]), comb[mt]);
                    if (has_mag) v = __fmul_rn(v, mg_cur[r]);
                    if (has_bias) v = __fadd_rn(v, bs_cur[r]);
                    if (SQRELU) {
                        v = v > 0.0f ? v : 0.0f;
                        v = __fmul_rn(v, v);
                    }
                    vb[u][mt][r] = v;
                    ab[u][mt][r] = av[r];
                }
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                mg_cur[r] = mg_nxt[r];
                bs_cur[r] = bs_nxt[r];
            }
        }
#pragma unroll
        for (int u = 0; u < kSkBatch; ++u) {
            const int ti = t0 + u;
            const int nb = tile_n0(ti);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int m = mt * 16 + li;
                const uint32_t e = static_cast<uint32_t>(m * pb.N + nb);
                const bool live = ti < my_tiles && m < M;
                if (VEC4) {
                    // N % 4 == 0: the lane's four outputs are one aligned vector, inside N
                    // exactly when its first one is
                    const bool ok = live && nb < pb.N;
                    if (ACC_OUT)
                        __builtin_amdgcn_raw_buffer_store_b128(
                            v4i{ab[u][mt][0], ab[u][mt][1], ab[u][mt][2], ab[u][mt][3]}, racc,
                            ok ? e * 4u : 0x80000000u, 0, 0);
                    if (y) {
                        const uint32_t off = ok ? e * ES : 0x80000000u;
                        if constexpr (YDT == NSOSX_F32)
                            __builtin_amdgcn_raw_buffer_store_b128(
                                v4i{(int)__float_as_uint(vb[u][mt][0]), (int)__float_as_uint(vb[u][mt][1]),
                                    (int)__float_as_uint(vb[u][mt][2]), (int)__float_as_uint(vb[u][mt][3])},
                                ry, off, 0, 0);
                        else
                            __builtin_amdgcn_raw_buffer_store_b64(
                                v2u{pack_bf16x2(vb[u][mt][0], vb[u][mt][1]),
                                    pack_bf16x2(vb[u][mt][2], vb[u][mt][3])},
                                ry, off, 0, 0);
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const bool ok = live && nb + r < pb.N;
                        const uint32_t er = e + r;
                        if (ACC_OUT)
                            __builtin_amdgcn_raw_buffer_store_b32(ab[u][mt][r], racc,
                                                                  ok ? er * 4u : 0x80000000u, 0, 0);
                        if (y) buf_store_act<YDT>(ry, ok ? er * ES : 0x80000000u, vb[u][mt][r]);
                    }
                }
            }
        }
    }
}

// Grouped decode GEMV for M >= 2 token rows, the groups skinny_group() accepts
// (the launch reserves 64 KB of LDS); the others are left to a grouped_gemv_kernel
// launch over the same groups.  The decision is uniform per workgroup.
template <int YDT, bool SQRELU>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void grouped_skinny_kernel(const nsosx_linear_view* views,
                                                             const int32_t* __restrict__ view_sel,
                                                             const int8_t* __restrict__ q,
                                                             int64_t q_stride, int q_div,
                                                             const float* __restrict__ act_scale,
                                                             int64_t scale_stride, int M, void* y,
                                                             int64_t y_stride) {
    extern __shared__ __align__(16) char lds_gsk[];
    const int g = blockIdx.y;
    const nsosx_linear_view v = views[view_sel ? view_sel[g] : g];
    char* yb = static_cast<char*>(y) + g * y_stride * (YDT == NSOSX_F32 ? 4 : 2);
    if (!skinny_group(v, yb)) return;
    GemvProblem pb{v.packed, v.magnitude, v.bias, v.weight_scale, v.outputs, v.inputs};
    // wave-uniform (readfirstlane): the tile loops then branch on scalars, with exact
    // memory wait counts
    const int wave_id = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    const int num_waves = gridDim.x * 4;
    const int gi = g / q_div;
    const int8_t* qg = q + gi * q_stride;
    const float* sg = act_scale + gi * scale_stride;
    if (pb.K == 1024)
        skinny_body<1, 4, YDT, false, SQRELU, true>(pb, qg, sg, M, yb, nullptr, wave_id, num_waves,
                                                     lds_gsk);
    else
        skinny_body<1, 8, YDT, false, SQRELU, true>(pb, qg, sg, M, yb, nullptr, wave_id, num_waves,
                                                     lds_gsk);
}

// NW waves per workgroup share one copy of the activation fragments: 4, or 8
// for two m tiles at K = 2048 (64 KB of fragments), so the LDS that caps the
// workgroups per CU at one still holds two waves per SIMD.
template <int MT, int LT, int YDT, bool ACC_OUT, int NW, bool ML>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2))) void skinny_kernel(
    GemvProblem pb, const int8_t* __restrict__ q, const float* __restrict__ act_scale, int M,
    void* y, int32_t* acc_out) {
    extern __shared__ __align__(16) char lds_sk[];
    // wave-uniform (readfirstlane): the tile loops then branch on scalars, with exact
    // memory wait counts
    const int wave_id = __builtin_amdgcn_readfirstlane(blockIdx.x * NW + (threadIdx.x >> 6));
    if ((pb.N & 3) == 0)
        skinny_body<MT, LT, YDT, ACC_OUT, false, true, ML>(pb, q, act_scale, M, y, acc_out,
                                                           wave_id, gridDim.x * NW, lds_sk);
    else
        skinny_body<MT, LT, YDT, ACC_OUT, false, false, ML>(pb, q, act_scale, M, y, acc_out,
                                                            wave_id, gridDim.x * NW, lds_sk);
}

template <int MT, int YDT, bool ML>
static void launch_skinny_lt(const GemvProblem& pb, const int8_t* q, const float* as, int M,
                             void* y, int32_t* acc, int tiles, hipStream_t st) {
    // about 8 waves per CU: two workgroups of 4 waves (32 KB of fragments), or one of 8
    // (64 KB); LDS = the fragments (M_pad x K bytes) + one tile per wave (16 rows of K / 4)
#define NSOSX_SK(LT, NW_)                                                                       \
    {                                                                                           \
        constexpr int NW = (NW_);                                                               \
        const int wgs = std::max(1, std::min((tiles + NW - 1) / NW, NW == 4 ? 512 : 256));      \
        const size_t lds = (size_t)MT * pb.K * 16 + (size_t)NW * 4 * pb.K;                     \
        if (acc)                                                                                \
            hipLaunchKernelGGL((skinny_kernel<MT, LT, YDT, true, NW, ML>), dim3(wgs), dim3(NW * 64), \
                               lds, st, pb, q, as, M, y, acc);                                  \
        else                                                                                    \
            hipLaunchKernelGGL((skinny_kernel<MT, LT, YDT, false, NW, ML>), dim3(wgs), dim3(NW * 64), \
                               lds, st, pb, q, as, M, y, acc);                                  \
    }
    // (K = 4096: 64 KB of fragments + 4 waves' 16 KB tiles already fill 128 KB of the
    // 160 KB, so it stays at one workgroup of 4 waves)
    if (pb.K == 1024) NSOSX_SK(4, 4)
    else if (pb.K == 2048) NSOSX_SK(8, MT == 1 ? 4 : 8)
    else NSOSX_SK(16, 4)
#undef NSOSX_SK
}

template <int YDT, bool ML = false>
static void launch_skinny_t(const GemvProblem& pb, const int8_t* q, const float* as, int M,
                            void* y, int32_t* acc, hipStream_t st) {
    const int tiles = (pb.N + 15) / 16;
    const int mt = (M + 15) / 16;
    if (mt == 1) launch_skinny_lt<1, YDT, ML>(pb, q, as, M, y, acc, tiles, st);
    else launch_skinny_lt<2, YDT, ML>(pb, q, as, M, y, acc, tiles, st);
}

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

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" int nsosx_quantize_act_i8(const void* x, int x_dtype, int M, int K, int bits,
                                     int rms_input, int8_t* q, float* act_scale,
                                     float* rms_workspace, void* stream) {
    if (!x || !q || !act_scale) return fail(NSOSX_ERR_INVALID, "quantize_act: null pointer");
    if (M <= 0 || K <= 0) return fail(NSOSX_ERR_INVALID, "quantize_act: M and K must be > 0");
    if (bits < 2 || bits > 8) return fail(NSOSX_ERR_INVALID, "quantize_act: bits must be in [2, 8]");
    if (!valid_dtype(x_dtype)) return fail(NSOSX_ERR_INVALID, "quantize_act: bad dtype");
    if (rms_input && !rms_workspace)
        return fail(NSOSX_ERR_INVALID, "quantize_act: rms_input needs rms_workspace");
    if ((int64_t)M * K > ((int64_t)1 << 40))
        return fail(NSOSX_ERR_OVERFLOW, "quantize_act: M*K too large");
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (x_dtype == NSOSX_F32)
        return launch_quantize<NSOSX_F32>(x, M, K, bits, rms_input, q, act_scale, rms_workspace, st);
    return launch_quantize<NSOSX_BF16>(x, M, K, bits, rms_input, q, act_scale, rms_workspace, st);
}

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
        if (y_dtype == NSOSX_F32) launch_skinny_t<NSOSX_F32>(pb, q, act_scale, M, y, acc_out, st);
        else launch_skinny_t<NSOSX_BF16>(pb, q, act_scale, M, y, acc_out, st);
    } else if (path == 0) {
        GemvProblem pb{packed, magnitude, bias, weight_scale, N, K};
        if (y_dtype == NSOSX_F32) launch_gemv_t<NSOSX_F32>(pb, q, act_scale, M, y, acc_out, st);
        else launch_gemv_t<NSOSX_BF16>(pb, q, act_scale, M, y, acc_out, st);
    } else {
        GemmProblem pb{packed, magnitude, bias, weight_scale, N, K};
        if (y_dtype == NSOSX_F32) launch_gemm_t<NSOSX_F32>(pb, q, act_scale, M, y, acc_out, st);
        else launch_gemm_t<NSOSX_BF16>(pb, q, act_scale, M, y, acc_out, st);
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
        if (y_dtype == NSOSX_F32)
            hipLaunchKernelGGL((grouped_skinny_kernel<NSOSX_F32, false>), gsk, block,
                               kGroupedSkinnyLds, st, views_dev, nullptr, q, q_stride, 1,
                               act_scale, scale_stride, M, y, y_stride);
        else
            hipLaunchKernelGGL((grouped_skinny_kernel<NSOSX_BF16, false>), gsk, block,
                               kGroupedSkinnyLds, st, views_dev, nullptr, q, q_stride, 1,
                               act_scale, scale_stride, M, y, y_stride);
    }
    if (M == 1) { NSOSX_GG(1, 0) }
    else if (M == 2) { NSOSX_GG(2, skip) }
    else if (M <= 4) { NSOSX_GG(4, skip) }
    else { NSOSX_GG(8, skip) }
#undef NSOSX_GG
    return check_launch("grouped_gemv");
}

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

extern "C" int nsosx_pack_mfma_layout(const uint32_t* packed, int64_t n_words, uint32_t* out,
                                      void* stream) {
    if (!packed || !out || n_words < 0)
        return fail(NSOSX_ERR_INVALID, "pack_mfma_layout: bad argument");
    if (n_words == 0) return NSOSX_OK;
    hipLaunchKernelGGL(pack_mfma_kernel, dim3((unsigned)((n_words + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), packed, n_words, out);
    return check_launch("pack_mfma_layout");
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
    if (skinny_ok(M, K, N)) {
        // decode batches: the skinny MFMA kernel on the same words
        GemvProblem pb{packed_mfma, magnitude, bias, weight_scale, N, K};
        hipStream_t st = static_cast<hipStream_t>(stream);
        if (y_dtype == NSOSX_F32) launch_skinny_t<NSOSX_F32, true>(pb, q, act_scale, M, y, acc_out, st);
        else launch_skinny_t<NSOSX_BF16, true>(pb, q, act_scale, M, y, acc_out, st);
        return check_launch("ternary_gemm_mfma");
    }
    const int tiles = ((N + kG3BN - 1) / kG3BN) * ((M + kG3BM - 1) / kG3BM);
    GemmProblem pb{packed_mfma, magnitude, bias, weight_scale, N, K};
    hipStream_t st = static_cast<hipStream_t>(stream);
#define NSOSX_GM(YDT, ACC)                                                                    \
    hipLaunchKernelGGL((gemm3_mfma_kernel<YDT, ACC>), dim3(tiles), dim3(kGemm3Threads), kGemm3Smem, \
                       st, pb, q, act_scale, M, y, acc_out);
    if (y_dtype == NSOSX_F32) {
        if (acc_out) { NSOSX_GM(NSOSX_F32, true) } else { NSOSX_GM(NSOSX_F32, false) }
    } else {
        if (acc_out) { NSOSX_GM(NSOSX_BF16, true) } else { NSOSX_GM(NSOSX_BF16, false) }
    }
#undef NSOSX_GM
    return check_launch("ternary_gemm_mfma");
}

extern "C" int nsosx_grouped_ternary_gemm_mfma(const nsosx_linear_view* views_dev, int experts,
                                               const int32_t* offsets, const int32_t* perm,
                                               int gather, const int8_t* q,
                                               const float* act_scale, int K, int N,
                                               int total_rows, int squared_relu, void* y,
                                               int y_dtype, void* stream) {
    if (!views_dev || !offsets || !q || !act_scale || !y || (gather && !perm))
        return fail(NSOSX_ERR_INVALID, "grouped_ternary_gemm_mfma: null pointer");
    if (experts <= 0 || experts > 1024 || K <= 0 || K % kG3BK || N <= 0 || total_rows < 0)
        return fail(NSOSX_ERR_INVALID,
                    "grouped_ternary_gemm_mfma: bad shape (K % 128 == 0, <= 1024 experts)");
    if (K > kMfmaLayoutMaxK)
        return fail(NSOSX_ERR_OVERFLOW, "grouped_ternary_gemm_mfma: K too large for the MFMA "
                                        "layout's 64x-scaled int32 sums");
    if (!valid_dtype(y_dtype))
        return fail(NSOSX_ERR_INVALID, "grouped_ternary_gemm_mfma: bad dtype");
    if (total_rows == 0) return NSOSX_OK;
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
    if (rows <= 0 || experts <= 0 || k <= 0 || k > 8 || k > experts || dim <= 0 || hidden <= 0 ||
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
