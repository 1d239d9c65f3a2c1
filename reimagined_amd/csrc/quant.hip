// BitLinear activation quantization on gfx950: the RMS_PERI row norm with the
// reference's in-order sum, and per-token absmax int8 codes.
//
// Reference semantics (OXN/nsos/ of vitorGgC569/reimagined):
//   quantization  src/bitlinear.cpp:240-291, src/bitlinear_quantize_avx2.cpp:65-103
//   RMS_PERI norm src/bitlinear.cpp:460-466, src/tensor.cpp:3455-3492
#include "bitlinear.hpp"

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
// sum + v * v with the square rounded first.  A bf16 value's square (at most 16
// significant bits) is exact in float, so one fused multiply-add rounds the same
// sum; an f32 square is rounded on its own, as the reference loop does.
template <int DT>
__device__ __forceinline__ float sq_add(float sum, float v) {
    if constexpr (DT == NSOSX_F32) return __fadd_rn(sum, __fmul_rn(v, v));
    else return __fmaf_rn(v, v, sum);
}

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
                for (int j = 0; j < PER; ++j) sum = sq_add<DT>(sum, v[u][j]);
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
                for (int j = 0; j < PER; ++j) sum = sq_add<DT>(sum, v[j]);
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
// (load8 and the one-row quantize_row_wg live in bitlinear.hpp: the decode
// projections of gemv.hip use them too.)
// ===========================================================================
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
// are those of quantize_rows_vec_kernel (a row's x * inv products are kept in
// registers for the codes), so the same bits.
// clamp127(rintf(t)) as the low byte of a float's bits: the clamp comes first
// (rounding a value inside [-127, 127] cannot leave it, and a NaN clamps to -127
// either way), then adding 1.5 * 2^23 rounds to an integer, ties to even, and
// leaves it in the low mantissa bits as two's complement.
__device__ __forceinline__ uint32_t code_bits(float t) {
    return __float_as_uint(__fadd_rn(clamp127(t), 12582912.0f));
}
// the low bytes of four code_bits words, a in byte 0
__device__ __forceinline__ uint32_t pack4_code_bits(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const uint32_t ab = __builtin_amdgcn_perm(b, a, 0x0c0c0400u);
    const uint32_t cd = __builtin_amdgcn_perm(d, c, 0x0c0c0400u);
    return __builtin_amdgcn_perm(cd, ab, 0x05040100u);
}

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
        // streaming loads: x is read once here, and should not displace the codes this
        // pass writes (the GEMM's input) from the L2 and the MALL (measured in the
        // config-4 layer: out_proj's GEMM 83 -> 80 us, the pass itself +0.5 us)
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int w = 0; w < NW; ++w)
                raw[r][c][w] = load_stream16(
                    reinterpret_cast<const uint32_t*>(src + c * (kWave * 8 * ES) + w * 16));
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
        float v[CH][8];  // the row's normalized values, kept for the codes
        float m = 0.0f;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            unpack(raw[r][c], v[c]);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (RMS) v[c][j] = __fmul_rn(v[c][j], inv);
                m = fmaxf(m, fabsf(v[c][j]));
            }
        }
        m = wave_max(m);
        if (row >= M) break;
        const float denom = __fadd_rn(m, 1e-8f);
        const float sc = __fdiv_rn(q_max, denom);
        if (lane == 0) act_scale[row] = __fdiv_rn(denom, q_max);
        int8_t* dst = q + (int64_t)row * K + lane * 8;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            uint32_t code[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) code[j] = code_bits(__fmul_rn(v[c][j], sc));
            *reinterpret_cast<uint2*>(dst + c * kWave * 8) =
                make_uint2(pack4_code_bits(code[0], code[1], code[2], code[3]),
                           pack4_code_bits(code[4], code[5], code[6], code[7]));
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

int launch_quantize_dt(const void* x, int dtype, int M, int K, int bits, int rms_input, int8_t* q,
                       float* act_scale, float* rms_ws, hipStream_t st) {
    if (dtype == NSOSX_F32)
        return launch_quantize<NSOSX_F32>(x, M, K, bits, rms_input, q, act_scale, rms_ws, st);
    return launch_quantize<NSOSX_BF16>(x, M, K, bits, rms_input, q, act_scale, rms_ws, st);
}

}  // namespace nsosx

using namespace nsosx;

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
