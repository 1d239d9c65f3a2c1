// fp32 linear algebra of the BitLinear float path and the packed STE backward.
//
//  * nsosx_linear_f32 -- the float reference path BitLinear keeps for
//    quantization-sensitive layers (src/bitlinear.cpp:465-518): optional
//    RMS_PERI input norm, y = x @ W^T, then * magnitude, then + bias.  The
//    faithful Mamba-2 block's B / C / dt projections and the MoE router's gate
//    run this way (src/mamba2.cpp:588-599, 655-662; src/jamba.cpp:8086-8098).
//  * nsosx_bitlinear_ste_backward -- BitLinear::backward on the packed path,
//    the straight-through estimator of src/bitlinear.cpp:1191-1357.
//
// Two kernel families:
//  * f32gemm_kernel: a 128 x 128 output block per workgroup of four waves, each
//    wave 64 x 64 as 2 x 2 tiles of v_mfma_f32_32x32x2_f32, 32-deep reduction
//    stages double-buffered in LDS (one barrier per stage).  Both operands are
//    staged reduction-major ([k][row] in LDS) whatever their layout in HBM;
//    the loader is a template: rows contiguous along the reduction (x, W, the
//    gradient as the left operand of d_act), rows contiguous along the output
//    (the gradient as the left operand of dW), int8 codes times a per-row
//    scale (the dequantized activations x_q * act_scale), or the packed
//    ternary codes decoded to {-1, 0, +1}.
//  * dot_kernel: one wave per row of the large operand for the skinny shapes
//    (router gates with N <= 16, decode with M <= 8), which leave an MFMA
//    block mostly empty; the wave holds its row's K-chunks and dots them with
//    the <= 16 rows of the small operand.
#include "common.hpp"

#include <cmath>

namespace nsosx {

typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kGB = 128;        // output block (rows and columns)
constexpr int kGK = 32;         // reduction depth of one LDS stage
constexpr int kGLd = kGB + 4;   // LDS row pitch in floats (keeps 16-byte alignment)
constexpr int kDotMax = 16;     // rows of the small operand in dot_kernel

// Operand layouts of f32gemm_kernel.  The output is [rows, cols] = [M, N]; the
// reduction runs over K.  "o" below is the operand's output index (m for the
// left operand, n for the right one), "k" the reduction index.
enum OperandKind {
    kRowK = 0,       // f32 [o][k] (row stride ld); optional per-o scale (RMS inverse)
    kRowKBf16 = 1,   // bf16 [o][k]; optional per-o scale
    kRowO = 2,       // f32 [k][o] (row stride ld)
    kCodes = 3,      // int8 [k][o] (row stride ld) times scale[k]: x_q * act_scale
    kTernary = 4,    // packed ternary [k][o / 16 words] (row stride ld words)
};

enum Epilogue {
    kEpiAffine = 0,  // * mag[n], + bias[n]; f32 or bf16 out
    kEpiScale = 1,   // * scale; f32 out
    kEpiClip = 2,    // 0 where |wlat[m,n] / scale| > 1 (the STE clip); f32 out
};

struct GemmArgs {
    const void* a;
    int64_t lda;
    const float* a_scale;
    const void* b;
    int64_t ldb;
    const float* b_scale;
    int M, N, K;
    const float* mag;
    const float* bias;
    void* y;
    int64_t ldy;
    int y_bf16;
    float scale;
    const float* wlat;
    int64_t ldw;
};

// Global -> registers: 16 floats per thread per stage, in the operand's own
// order; st_tile() writes them reduction-major into the LDS stage.
template <int KIND>
__device__ __forceinline__ void ld_tile(const void* __restrict__ src, int64_t ld,
                                        const float* __restrict__ scale, int o0, int k0, int O,
                                        int Kr, float (&r)[16]) {
    const int t = threadIdx.x;
    if constexpr (KIND == kRowK || KIND == kRowKBf16) {
        const int kq = (t & 7) * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int o = o0 + (t >> 3) + 32 * i;
            const int k = k0 + kq;
            float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (o < O && k < Kr) {
                if constexpr (KIND == kRowK) {
                    const float4 f = *reinterpret_cast<const float4*>(
                        static_cast<const float*>(src) + (int64_t)o * ld + k);
                    v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
                } else {
                    const uint2 h = *reinterpret_cast<const uint2*>(
                        static_cast<const uint16_t*>(src) + (int64_t)o * ld + k);
                    v[0] = __uint_as_float(h.x << 16);
                    v[1] = __uint_as_float(h.x & 0xffff0000u);
                    v[2] = __uint_as_float(h.y << 16);
                    v[3] = __uint_as_float(h.y & 0xffff0000u);
                }
                if (scale) {
                    const float s = scale[o];
#pragma unroll
                    for (int c = 0; c < 4; ++c) v[c] = __fmul_rn(v[c], s);
                }
            }
#pragma unroll
            for (int c = 0; c < 4; ++c) r[4 * i + c] = v[c];
        }
    } else if constexpr (KIND == kRowO) {
        const int oq = (t & 31) * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int k = k0 + (t >> 5) + 8 * i;
            const int o = o0 + oq;
            float4 f = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (k < Kr && o < O)
                f = *reinterpret_cast<const float4*>(static_cast<const float*>(src) +
                                                      (int64_t)k * ld + o);
            r[4 * i + 0] = f.x; r[4 * i + 1] = f.y; r[4 * i + 2] = f.z; r[4 * i + 3] = f.w;
        }
    } else if constexpr (KIND == kCodes) {
        const int k = k0 + (t >> 3);
        const int o = o0 + (t & 7) * 16;
        uint4 w = make_uint4(0u, 0u, 0u, 0u);
        float s = 0.0f;
        if (k < Kr && o < O) {
            w = *reinterpret_cast<const uint4*>(static_cast<const int8_t*>(src) + (int64_t)k * ld +
                                                o);
            s = scale[k];
        }
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int8_t c = static_cast<int8_t>((ws[i >> 2] >> (8 * (i & 3))) & 0xffu);
            r[i] = __fmul_rn(static_cast<float>(c), s);
        }
    } else {  // kTernary
        const int k = k0 + (t >> 3);
        const int o = o0 + (t & 7) * 16;
        uint32_t w = 0x55555555u;  // code 1 = 0
        if (k < Kr && o < O) w = static_cast<const uint32_t*>(src)[(int64_t)k * ld + (o >> 4)];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t c = (w >> (2 * i)) & 3u;
            r[i] = c == 0u ? -1.0f : (c == 2u ? 1.0f : 0.0f);
        }
    }
}

template <int KIND>
__device__ __forceinline__ void st_tile(float* __restrict__ s, const float (&r)[16]) {
    const int t = threadIdx.x;
    if constexpr (KIND == kRowK || KIND == kRowKBf16) {
        const int kq = (t & 7) * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int o = (t >> 3) + 32 * i;
#pragma unroll
            for (int c = 0; c < 4; ++c) s[(kq + c) * kGLd + o] = r[4 * i + c];
        }
    } else if constexpr (KIND == kRowO) {
        const int oq = (t & 31) * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int k = (t >> 5) + 8 * i;
            *reinterpret_cast<float4*>(s + k * kGLd + oq) =
                make_float4(r[4 * i], r[4 * i + 1], r[4 * i + 2], r[4 * i + 3]);
        }
    } else {  // kCodes / kTernary: one reduction row, 16 consecutive outputs
        const int k = t >> 3;
        const int o = (t & 7) * 16;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *reinterpret_cast<float4*>(s + k * kGLd + o + 4 * i) =
                make_float4(r[4 * i], r[4 * i + 1], r[4 * i + 2], r[4 * i + 3]);
    }
}

template <int AK, int BK, int EPI>
__global__ __launch_bounds__(256, 2) void f32gemm_kernel(GemmArgs g) {
    __shared__ __align__(16) float sA[2][kGK * kGLd];
    __shared__ __align__(16) float sB[2][kGK * kGLd];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.x * kGB, n0 = blockIdx.y * kGB;
    const int stages = (g.K + kGK - 1) / kGK;

    v16f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    float ra[16], rb[16];
    ld_tile<AK>(g.a, g.lda, g.a_scale, m0, 0, g.M, g.K, ra);
    ld_tile<BK>(g.b, g.ldb, g.b_scale, n0, 0, g.N, g.K, rb);
    st_tile<AK>(sA[0], ra);
    st_tile<BK>(sB[0], rb);
    __syncthreads();

    const int fr = lane >> 5;   // reduction row of this lane's fragment element
    const int fc = lane & 31;   // output index within a 32-wide tile
    for (int st = 0; st < stages; ++st) {
        const int cur = st & 1;
        const bool more = st + 1 < stages;
        if (more) {
            ld_tile<AK>(g.a, g.lda, g.a_scale, m0, (st + 1) * kGK, g.M, g.K, ra);
            ld_tile<BK>(g.b, g.ldb, g.b_scale, n0, (st + 1) * kGK, g.N, g.K, rb);
        }
        const float* a = sA[cur] + wm * 64 + fc;
        const float* b = sB[cur] + wn * 64 + fc;
#pragma unroll
        for (int kk = 0; kk < kGK; kk += 2) {
            const int off = (kk + fr) * kGLd;
            const float a0 = a[off], a1 = a[off + 32];
            const float b0 = b[off], b1 = b[off + 32];
            acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b0, acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b1, acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b0, acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b1, acc[1][1], 0, 0, 0);
        }
        if (more) {
            // the other buffer was last read before the previous stage's barrier
            st_tile<AK>(sA[cur ^ 1], ra);
            st_tile<BK>(sB[cur ^ 1], rb);
        }
        __syncthreads();
    }

    // C tile layout of the 32x32 MFMA: register r of lane l holds
    // row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
            const int n = n0 + wn * 64 + ni * 32 + fc;
            if (n >= g.N) continue;
            float mg = 1.0f, bs = 0.0f;
            if constexpr (EPI == kEpiAffine) {
                if (g.mag) mg = g.mag[n];
                if (g.bias) bs = g.bias[n];
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * 64 + mi * 32 + 8 * (r >> 2) + 4 * fr + (r & 3);
                if (m >= g.M) continue;
                float v = acc[mi][ni][r];
                if constexpr (EPI == kEpiAffine) {
                    if (g.mag) v = __fmul_rn(v, mg);
                    if (g.bias) v = __fadd_rn(v, bs);
                    if (g.y_bf16)
                        static_cast<uint16_t*>(g.y)[(int64_t)m * g.ldy + n] = f32_to_bf16(v);
                    else
                        static_cast<float*>(g.y)[(int64_t)m * g.ldy + n] = v;
                } else if constexpr (EPI == kEpiScale) {
                    static_cast<float*>(g.y)[(int64_t)m * g.ldy + n] = __fmul_rn(v, g.scale);
                } else {
                    const float wv = g.wlat[(int64_t)m * g.ldw + n];
                    static_cast<float*>(g.y)[(int64_t)m * g.ldy + n] =
                        fabsf(__fdiv_rn(wv, g.scale)) > 1.0f ? 0.0f : v;
                }
            }
        }
}

template <int AK, int BK, int EPI>
static void launch_f32gemm(const GemmArgs& g, hipStream_t st) {
    const dim3 grid((g.M + kGB - 1) / kGB, (g.N + kGB - 1) / kGB);
    hipLaunchKernelGGL((f32gemm_kernel<AK, BK, EPI>), grid, dim3(256), 0, st, g);
}

// ---------------------------------------------------------------------------
// Skinny shapes: one wave per row of the big operand.
//   PER_M: wave m holds x[m] (times inv[m]) and dots it with the N <= 16 rows
//          of W (router gates);
//   else : wave n holds W[n] and dots it with the M <= 16 rows of x (decode).
// ---------------------------------------------------------------------------
template <int XDT, bool PER_M, int JM>
__global__ __launch_bounds__(256) void dot_kernel(const void* __restrict__ x,
                                                  const float* __restrict__ inv,
                                                  const float* __restrict__ w, int M, int N,
                                                  int K, const float* __restrict__ mag,
                                                  const float* __restrict__ bias, void* y,
                                                  int y_bf16) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int nbig = PER_M ? M : N;
    const int nsmall = PER_M ? N : M;
    if (row >= nbig) return;
    float acc[JM];
#pragma unroll
    for (int j = 0; j < JM; ++j) acc[j] = 0.0f;
    // four consecutive k per lane per step (K % 4 == 0, 16-byte aligned rows), so a
    // step's loads are 16 bytes wide; with at most 4 small rows the loads of U = 4
    // steps (a row of 1024) are issued together, small rows past nsmall and steps
    // past K re-reading valid addresses (their products are not added)
    auto load4 = [&](const void* base, int dt, int64_t off, float v[4]) {
        if (dt == NSOSX_F32) {
            const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + off);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        } else {
            const uint2 a = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + off);
            v[0] = __uint_as_float(a.x << 16); v[1] = __uint_as_float(a.x & 0xFFFF0000u);
            v[2] = __uint_as_float(a.y << 16); v[3] = __uint_as_float(a.y & 0xFFFF0000u);
        }
    };
    auto xval4 = [&](int m, int k, float v[4]) {
        load4(x, XDT, (int64_t)m * K + k, v);
        if (inv) {
            const float s = inv[m];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = __fmul_rn(v[e], s);
        }
    };
    constexpr int U = JM <= 4 ? 4 : 1;
    for (int k0 = 4 * lane; k0 < K; k0 += 256 * U) {
        float mine[U][4], other[U][JM][4];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = min(k0 + 256 * u, K - 4);
            if (PER_M) xval4(row, k, mine[u]);
            else load4(w, NSOSX_F32, (int64_t)row * K + k, mine[u]);
#pragma unroll
            for (int j = 0; j < JM; ++j) {
                const int jj = min(j, nsmall - 1);
                if (PER_M) load4(w, NSOSX_F32, (int64_t)jj * K + k, other[u][j]);
                else xval4(jj, k, other[u][j]);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (k0 + 256 * u >= K) break;
#pragma unroll
            for (int j = 0; j < JM; ++j)
                if (j < nsmall)
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[j] = __fmaf_rn(mine[u][e], other[u][j][e], acc[j]);
        }
    }
#pragma unroll
    for (int j = 0; j < JM; ++j) {
        if (j >= nsmall) continue;
        float v = acc[j];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v = __fadd_rn(v, __shfl_xor(v, off));
        if (lane == 0) {
            const int m = PER_M ? row : j;
            const int n = PER_M ? j : row;
            if (mag) v = __fmul_rn(v, mag[n]);
            if (bias) v = __fadd_rn(v, bias[n]);
            if (y_bf16) static_cast<uint16_t*>(y)[(int64_t)m * N + n] = f32_to_bf16(v);
            else static_cast<float*>(y)[(int64_t)m * N + n] = v;
        }
    }
}

// ---------------------------------------------------------------------------
// Skinny outputs over many rows (N <= 64, M > kDotMax: the faithful Mamba-2
// block's B / C / dt projections, router gates at prefill).  A workgroup of
// four waves owns 32 rows x all N columns as 2 x NT tiles of
// v_mfma_f32_16x16x4f32 and splits K among its waves: 32-deep slice s goes to
// wave s % 4, x streaming from HBM and W (at most 64 x K floats) from L2, the
// next slice's loads in flight while the current one is contracted.  Lane l
// loads, for each of its rows (l % 16) + 16 i and columns (l % 16) + 16 j, the
// eight elements k0 + 8 (l / 16) .. + 7 (two 16-byte loads per row, so a row's
// four lanes read 128 contiguous bytes); MFMA step e (0..7) contracts, in lane
// group l / 16, element k0 + 8 (l / 16) + e of both operands.  The D tile of a
// 16x16x4 MFMA leaves row 4 (l / 16) + r, column l % 16 in register r.  The four
// waves' partial tiles are added in wave order through LDS by wave 0.
// ---------------------------------------------------------------------------
typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int kSkinnyRows = 32;   // rows per workgroup
constexpr int kSkinnyMaxN = 64;
constexpr int kSkinnyWaves = 4;   // K split

template <int XDT>
__device__ __forceinline__ void load8(const void* p, int64_t i, float v[8]) {
    if constexpr (XDT == NSOSX_F32) {
        const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
        const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
        const u32x4 u = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(p) + i);
        const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[2 * j] = __uint_as_float(wd[j] << 16);
            v[2 * j + 1] = __uint_as_float(wd[j] & 0xFFFF0000u);
        }
    }
}

template <int XDT, int NT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NT <= 2 ? 2 : 3))) void skinny_f32_kernel(const void* __restrict__ x, int rms,
                                                     float eps, const float* __restrict__ w, int M,
                                                     int N, int K, const float* __restrict__ mag,
                                                     const float* __restrict__ bias, void* y,
                                                     int y_bf16) {
    __shared__ __align__(16) v4f s_part[kSkinnyWaves - 1][2 * NT][64];
    __shared__ float s_ss[kSkinnyWaves][kSkinnyRows];  // per-wave sums of squares by row
    __shared__ float s_inv[kSkinnyRows];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int r0 = blockIdx.x * kSkinnyRows;
    int64_t abase[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = min(r0 + lr + 16 * i, M - 1);  // rows past M are computed, not stored
        abase[i] = (int64_t)r * K;
    }
    float ss[2] = {0.0f, 0.0f};  // RMS_PERI: the lane's share of its rows' sums of squares
    int64_t bbase[NT];
    bool bok[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int n = lr + 16 * j;
        bok[j] = n < N;
        bbase[j] = (int64_t)min(n, N - 1) * K;
    }
    // one slice of both operands: K % 4 == 0, so each 4-element half of a lane's
    // eight is wholly in or out; columns past N contract zeros
    auto load_slice = [&](int k0, float (&a)[2][8], float (&b)[NT][8]) {
        const int kk = k0 + 8 * lg;
        const bool in0 = kk < K, in1 = kk + 4 < K;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            if (in1) {
                load8<XDT>(x, abase[i] + kk, a[i]);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    a[i][e] = (e < 4 && in0) ? load_act<XDT>(x, abase[i] + kk + e) : 0.0f;
            }
        }
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            if (in1 && bok[j]) {
                load8<NSOSX_F32>(w, bbase[j] + kk, b[j]);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    b[j][e] = (e < 4 && in0 && bok[j]) ? w[bbase[j] + kk + e] : 0.0f;
            }
        }
    };
    v4f acc[2][NT];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    auto contract = [&](const float (&a)[2][8], const float (&b)[NT][8]) {
        if (rms) {
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int e = 0; e < 8; ++e) ss[i] = __fmaf_rn(a[i][e], a[i][e], ss[i]);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < NT; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][e], b[j][e], acc[i][j],
                                                                     0, 0, 0);
    };
    // slices wave, wave + 4, ... (slices past K load nothing and contract zeros).  Up to
    // two column tiles: two register sets, the next slice loading while the current one
    // is contracted.  Three or four: one set (the loads' latency is covered by the other
    // workgroups' waves on the SIMD, which two sets of NT = 4 would not leave room for).
    constexpr int kStride = 32 * kSkinnyWaves;
    float a0[2][8], b0[NT][8];
    int k0 = 32 * wave;
    if constexpr (NT <= 2) {
        float a1[2][8], b1[NT][8];
        load_slice(k0, a0, b0);
        for (; k0 < K; k0 += 2 * kStride) {
            load_slice(k0 + kStride, a1, b1);
            contract(a0, b0);
            load_slice(k0 + 2 * kStride, a0, b0);
            contract(a1, b1);
        }
    } else {
        for (; k0 < K; k0 += kStride) {
            load_slice(k0, a0, b0);
            contract(a0, b0);
        }
    }
    if (wave > 0) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < NT; ++j) s_part[wave - 1][i * NT + j][lane] = acc[i][j];
    }
    if (rms) {
        // the row's four lane groups, then its four waves
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            ss[i] += __shfl_xor(ss[i], 16);
            ss[i] += __shfl_xor(ss[i], 32);
            if (lg == 0) s_ss[wave][lr + 16 * i] = ss[i];
        }
    }
    __syncthreads();
    if (wave > 0) return;
    if (rms && lane < kSkinnyRows) {
        const float t = ((s_ss[0][lane] + s_ss[1][lane]) + s_ss[2][lane]) + s_ss[3][lane];
        s_inv[lane] = __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(t, static_cast<float>(K)), eps)));
    }
    asm volatile("" ::: "memory");  // LDS operations of one wave complete in order
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int v = 0; v < kSkinnyWaves - 1; ++v) acc[i][j] += s_part[v][i * NT + j][lane];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int n = lr + 16 * j;
        if (n >= N) continue;
        const float mg = mag ? mag[n] : 1.0f;
        const float bs = bias ? bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = r0 + 16 * i + 4 * lg + r;
                if (m >= M) continue;
                float v = acc[i][j][r];
                if (rms) v = __fmul_rn(v, s_inv[16 * i + 4 * lg + r]);
                if (mag) v = __fmul_rn(v, mg);
                if (bias) v = __fadd_rn(v, bs);
                if (y_bf16) static_cast<uint16_t*>(y)[(int64_t)m * N + n] = f32_to_bf16(v);
                else static_cast<float*>(y)[(int64_t)m * N + n] = v;
            }
    }
}

template <int XDT>
static void launch_skinny(const void* x, int rms, const float* w, int M, int N, int K,
                          const float* mag, const float* bias, void* y, int ybf, hipStream_t st) {
    const float eps = 1e-6f;
    const dim3 grid((M + kSkinnyRows - 1) / kSkinnyRows);
    switch ((N + 15) / 16) {
        case 1: hipLaunchKernelGGL((skinny_f32_kernel<XDT, 1>), grid, dim3(256), 0, st, x, rms, eps, w,
                                   M, N, K, mag, bias, y, ybf); break;
        case 2: hipLaunchKernelGGL((skinny_f32_kernel<XDT, 2>), grid, dim3(256), 0, st, x, rms, eps, w,
                                   M, N, K, mag, bias, y, ybf); break;
        case 3: hipLaunchKernelGGL((skinny_f32_kernel<XDT, 3>), grid, dim3(256), 0, st, x, rms, eps, w,
                                   M, N, K, mag, bias, y, ybf); break;
        default: hipLaunchKernelGGL((skinny_f32_kernel<XDT, 4>), grid, dim3(256), 0, st, x, rms, eps, w,
                                    M, N, K, mag, bias, y, ybf); break;
    }
}

// ---------------------------------------------------------------------------
// STE backward pieces.
// ---------------------------------------------------------------------------
constexpr int kColRows = 256;   // rows per partial of the column reductions

// partial[c][j]: over rows [c*kColRows, ...) of column j, sum grad*pre and
// sum grad; gp[i,j] = grad*mag[j] (written over pre when mag is given).
__global__ __launch_bounds__(256) void colred_kernel(const float* __restrict__ grad,
                                                     float* __restrict__ pre_gp,
                                                     const float* __restrict__ mag, int M, int N,
                                                     float* __restrict__ part_mag,
                                                     float* __restrict__ part_bias) {
    const int j = blockIdx.x * 256 + threadIdx.x;
    const int c = blockIdx.y;
    if (j >= N) return;
    const int i0 = c * kColRows, i1 = min(M, i0 + kColRows);
    float sm = 0.0f, sb = 0.0f;
    const float mg = mag ? mag[j] : 1.0f;
    for (int i = i0; i < i1; ++i) {
        const float g = grad[(int64_t)i * N + j];
        if (mag) {
            const float p = pre_gp[(int64_t)i * N + j];
            sm = __fadd_rn(sm, __fmul_rn(g, p));
            pre_gp[(int64_t)i * N + j] = __fmul_rn(g, mg);
        }
        sb = __fadd_rn(sb, g);
    }
    if (part_mag) part_mag[(int64_t)c * N + j] = sm;
    if (part_bias) part_bias[(int64_t)c * N + j] = sb;
}

__global__ __launch_bounds__(256) void colred_finish_kernel(const float* __restrict__ part,
                                                            int chunks, int N,
                                                            float* __restrict__ out) {
    const int j = blockIdx.x * 256 + threadIdx.x;
    if (j >= N) return;
    float s = 0.0f;
    for (int c = 0; c < chunks; ++c) s = __fadd_rn(s, part[(int64_t)c * N + j]);
    out[j] = s;
}

// Tensor::rmsnorm_backward (src/tensor.cpp:3997-4056) with x_norm = x * inv:
// dot = sum_k g*y / K; dx = (g - y*dot) * inv.  One wave per row.
template <int XDT>
__global__ __launch_bounds__(256) void rms_backward_kernel(const void* __restrict__ x,
                                                           const float* __restrict__ inv,
                                                           const float* __restrict__ g, int M,
                                                           int K, float* __restrict__ dx) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    const float s = inv[row];
    const int64_t base = (int64_t)row * K;
    float dot = 0.0f;
    for (int k = lane; k < K; k += 64) {
        const float yv = __fmul_rn(load_act<XDT>(x, base + k), s);
        dot = __fmaf_rn(g[base + k], yv, dot);
    }
    for (int off = 32; off > 0; off >>= 1) dot = __fadd_rn(dot, __shfl_xor(dot, off));
    dot = __fdiv_rn(dot, static_cast<float>(K));
    for (int k = lane; k < K; k += 64) {
        const float yv = __fmul_rn(load_act<XDT>(x, base + k), s);
        dx[base + k] = __fmul_rn(__fmaf_rn(-yv, dot, g[base + k]), s);
    }
}

static int64_t round256(int64_t v) { return (v + 255) & ~int64_t(255); }

struct SteWorkspace {
    float* gp;        // [M, N]: pre, then grad * magnitude
    float* dact;      // [M, K] (rms_input only)
    float* inv;       // [M] (rms_input only)
    float* part;      // [chunks, N] x 2
    int64_t bytes;
};

static SteWorkspace ste_layout(void* base, int M, int K, int N, int rms_input) {
    SteWorkspace w{};
    const int chunks = (M + kColRows - 1) / kColRows;
    int64_t off = 0;
    auto take = [&](int64_t n) {
        float* p = base ? reinterpret_cast<float*>(static_cast<char*>(base) + off) : nullptr;
        off += round256(n * (int64_t)sizeof(float));
        return p;
    };
    w.gp = take((int64_t)M * N);
    w.dact = rms_input ? take((int64_t)M * K) : nullptr;
    w.inv = rms_input ? take(M) : nullptr;
    w.part = take(2 * (int64_t)chunks * N);
    w.bytes = off;
    return w;
}

}  // namespace nsosx

using namespace nsosx;

extern "C" int nsosx_linear_f32(const void* x, int x_dtype, int M, int K, const float* w, int N,
                                int rms_input, const float* magnitude, const float* bias, void* y,
                                int y_dtype, float* rms_workspace, void* stream) {
    if (!x || !w || !y) return fail(NSOSX_ERR_INVALID, "linear_f32: null pointer");
    if (M <= 0 || K <= 0 || N <= 0) return fail(NSOSX_ERR_INVALID, "linear_f32: empty shape");
    if (K % 4 != 0) return fail(NSOSX_ERR_INVALID, "linear_f32: K must be a multiple of 4");
    if (!valid_dtype(x_dtype) || !valid_dtype(y_dtype))
        return fail(NSOSX_ERR_INVALID, "linear_f32: bad dtype");
    if (rms_input && !rms_workspace)
        return fail(NSOSX_ERR_INVALID, "linear_f32: rms_input needs rms_workspace");
    if ((int64_t)M * K > ((int64_t)1 << 40) || (int64_t)M * N > ((int64_t)1 << 40))
        return fail(NSOSX_ERR_OVERFLOW, "linear_f32: size too large");
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(w) % 16)
        return fail(NSOSX_ERR_INVALID, "linear_f32: x and w must be 16-byte aligned");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int ybf = y_dtype == NSOSX_BF16;
    // Skinny outputs over many rows: one pass over x, the RMS_PERI sums of squares taken
    // on the way and the 1 / rms applied to the row's dot products (equal to the dot of
    // the normalised row to rounding; bf16 rows are read 16 bytes at a time: K % 8 keeps
    // them aligned)
    if (N <= kSkinnyMaxN && M > kDotMax && (x_dtype == NSOSX_F32 || K % 8 == 0)) {
        if (x_dtype == NSOSX_F32)
            launch_skinny<NSOSX_F32>(x, rms_input, w, M, N, K, magnitude, bias, y, ybf, st);
        else
            launch_skinny<NSOSX_BF16>(x, rms_input, w, M, N, K, magnitude, bias, y, ybf, st);
        return check_launch("linear_f32");
    }
    if (rms_input) launch_rms_inv(x, x_dtype, M, K, 1e-6f, rms_workspace, st);
    const float* inv = rms_input ? rms_workspace : nullptr;
    if (N <= kDotMax || M <= kDotMax) {
        const bool per_m = N <= kDotMax && !(M <= kDotMax && M < N);
        const int rows = per_m ? M : N;
        const dim3 grid((rows + 3) / 4);
        const int nsmall = per_m ? N : M;
#define NSOSX_DOT(XDT, PM, JM)                                                                \
    hipLaunchKernelGGL((dot_kernel<XDT, PM, JM>), grid, dim3(256), 0, st, x, inv, w, M, N, K, \
                       magnitude, bias, y, ybf)
#define NSOSX_DOT_J(XDT, PM)                                                 \
    if (nsmall == 1) NSOSX_DOT(XDT, PM, 1);                                  \
    else if (nsmall <= 4) NSOSX_DOT(XDT, PM, 4);                             \
    else NSOSX_DOT(XDT, PM, kDotMax);
        if (x_dtype == NSOSX_F32) {
            if (per_m) { NSOSX_DOT_J(NSOSX_F32, true) } else { NSOSX_DOT_J(NSOSX_F32, false) }
        } else {
            if (per_m) { NSOSX_DOT_J(NSOSX_BF16, true) } else { NSOSX_DOT_J(NSOSX_BF16, false) }
        }
#undef NSOSX_DOT_J
#undef NSOSX_DOT
        return check_launch("linear_f32");
    }
    GemmArgs g{};
    g.a = x; g.lda = K; g.a_scale = inv;
    g.b = w; g.ldb = K; g.b_scale = nullptr;
    g.M = M; g.N = N; g.K = K;
    g.mag = magnitude; g.bias = bias; g.y = y; g.ldy = N; g.y_bf16 = ybf;
    if (x_dtype == NSOSX_F32) launch_f32gemm<kRowK, kRowK, kEpiAffine>(g, st);
    else launch_f32gemm<kRowKBf16, kRowK, kEpiAffine>(g, st);
    return check_launch("linear_f32");
}

extern "C" int64_t nsosx_bitlinear_ste_backward_workspace(int M, int K, int N, int rms_input) {
    if (M <= 0 || K <= 0 || N <= 0) return 0;
    return ste_layout(nullptr, M, K, N, rms_input).bytes;
}

extern "C" int nsosx_bitlinear_ste_backward(const void* x, int x_dtype, const int8_t* q,
                                            const float* act_scale, const float* w_latent,
                                            const uint32_t* packed, float weight_scale, int M,
                                            int K, int N, int rms_input, const float* magnitude,
                                            const float* grad, float* dx, float* dW, float* dmag,
                                            float* dbias, void* workspace, void* stream) {
    if (!q || !act_scale || !w_latent || !packed || !grad || !dx || !dW || !workspace)
        return fail(NSOSX_ERR_INVALID, "bitlinear_ste_backward: null pointer");
    if (rms_input && !x)
        return fail(NSOSX_ERR_INVALID, "bitlinear_ste_backward: rms_input needs the input x");
    if (dmag && !magnitude)
        return fail(NSOSX_ERR_INVALID, "bitlinear_ste_backward: dmag needs the magnitude");
    if (M <= 0 || K <= 0 || N <= 0)
        return fail(NSOSX_ERR_INVALID, "bitlinear_ste_backward: empty shape");
    if (K % 16 != 0 || N % 4 != 0)
        return fail(NSOSX_ERR_INVALID,
                    "bitlinear_ste_backward: K must be a multiple of 16 and N of 4");
    if (!valid_dtype(x_dtype)) return fail(NSOSX_ERR_INVALID, "bitlinear_ste_backward: bad dtype");
    if (!(weight_scale > 0.0f) || !std::isfinite(weight_scale))
        return fail(NSOSX_ERR_INVALID, "bitlinear_ste_backward: weight_scale must be finite > 0");
    if ((int64_t)M * K > ((int64_t)1 << 40) || (int64_t)M * N > ((int64_t)1 << 40) ||
        (int64_t)N * K > ((int64_t)1 << 40))
        return fail(NSOSX_ERR_OVERFLOW, "bitlinear_ste_backward: size too large");
    if (reinterpret_cast<uintptr_t>(q) % 16 || reinterpret_cast<uintptr_t>(grad) % 16 ||
        reinterpret_cast<uintptr_t>(workspace) % 256)
        return fail(NSOSX_ERR_INVALID,
                    "bitlinear_ste_backward: q and grad 16-byte, workspace 256-byte aligned");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const SteWorkspace ws = ste_layout(workspace, M, K, N, rms_input);
    const int chunks = (M + kColRows - 1) / kColRows;
    float* part_mag = ws.part;
    float* part_bias = ws.part + (int64_t)chunks * N;

    // pre = acc * (act_scale * weight_scale), the un-fused GEMM output (bitlinear.cpp:1267-1275)
    if (magnitude) {
        int rc = nsosx_ternary_gemm(q, act_scale, packed, weight_scale, M, K, N, nullptr, nullptr,
                                    ws.gp, NSOSX_F32, nullptr, stream);
        if (rc) return rc;
    }
    if (magnitude || dbias) {
        const dim3 grid((N + 255) / 256, chunks);
        hipLaunchKernelGGL(colred_kernel, grid, dim3(256), 0, st, grad, ws.gp, magnitude, M, N,
                           dmag ? part_mag : nullptr, dbias ? part_bias : nullptr);
        if (dmag)
            hipLaunchKernelGGL(colred_finish_kernel, dim3((N + 255) / 256), dim3(256), 0, st,
                               part_mag, chunks, N, dmag);
        if (dbias)
            hipLaunchKernelGGL(colred_finish_kernel, dim3((N + 255) / 256), dim3(256), 0, st,
                               part_bias, chunks, N, dbias);
    }
    const float* gp = magnitude ? ws.gp : grad;

    // dW = gp^T @ (x_q * act_scale), zero where |W / (ws + 1e-8f)| > 1 (bitlinear.cpp:1293-1321)
    GemmArgs gw{};
    gw.a = gp; gw.lda = N; gw.a_scale = nullptr;
    gw.b = q; gw.ldb = K; gw.b_scale = act_scale;
    gw.M = N; gw.N = K; gw.K = M;
    gw.y = dW; gw.ldy = K; gw.scale = weight_scale + 1e-8f; gw.wlat = w_latent; gw.ldw = K;
    launch_f32gemm<kRowO, kCodes, kEpiClip>(gw, st);

    // d_act = gp @ (ternary * weight_scale) (bitlinear.cpp:1340)
    float* dact = rms_input ? ws.dact : dx;
    GemmArgs gd{};
    gd.a = gp; gd.lda = N; gd.a_scale = nullptr;
    gd.b = packed; gd.ldb = K / 16; gd.b_scale = nullptr;
    gd.M = M; gd.N = K; gd.K = N;
    gd.y = dact; gd.ldy = K; gd.scale = weight_scale;
    launch_f32gemm<kRowK, kTernary, kEpiScale>(gd, st);

    // dx = rmsnorm_backward(x, d_act, x_norm) (bitlinear.cpp:1352-1355)
    if (rms_input) {
        launch_rms_inv(x, x_dtype, M, K, 1e-6f, ws.inv, st);
        const dim3 grid((M + 3) / 4);
        if (x_dtype == NSOSX_F32)
            hipLaunchKernelGGL((rms_backward_kernel<NSOSX_F32>), grid, dim3(256), 0, st, x, ws.inv,
                               dact, M, K, dx);
        else
            hipLaunchKernelGGL((rms_backward_kernel<NSOSX_BF16>), grid, dim3(256), 0, st, x,
                               ws.inv, dact, M, K, dx);
    }
    return check_launch("bitlinear_ste_backward");
}
