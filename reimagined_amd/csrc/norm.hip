// Row norms around the hybrid block and the decode conv ring on gfx950.
//
// Reference semantics (OXN/nsos/ of vitorGgC569/reimagined):
//   Tensor::rmsnorm        src/tensor.cpp:3455-3492   inv = 1/sqrt(sum x^2 / K + eps), x * inv
//   Tensor::silu_gate      src/tensor.cpp:3323-3343   y * silu(z), silu split on the sign (3261-3282)
//   gated RMSNorm epilogue src/mamba2.cpp:2677-2680   RMSNorm(y * SiLU(z)) * gamma
//                          (GPU twin mamba_gated_rmsnorm_kernel, src/cuda/mamba_kernels.cu:3421-3445)
//   block composition      src/jamba.cpp:3158-3375    r = x + core; rmsnorm(r) [* gamma]
//   decode conv ring       src/mamba2.cpp:4072-4090   (GPU twin mamba2_faithful_conv_step_kernel,
//                          src/cuda/mamba_kernels.cu:3332-3358)
//
// The row sum of squares is a wave tree reduction in fp32 (as the reference's
// GPU kernels reduce); the CPU reference sums in index order, so outputs agree
// to float rounding of that sum, not bit for bit.
#include "common.hpp"

#include <cmath>

namespace nsosx {

// ===========================================================================
// out = (g * inv) * gamma with g = y * silu(z) (GATED) or g = y, one wave per
// row, two passes over the row (the second recomputes g).
// ===========================================================================
template <int DT, int ODT, bool GATED>
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(const void* __restrict__ y,
                                                           const void* __restrict__ z,
                                                           const float* __restrict__ gamma,
                                                           int rows, int dim, float eps,
                                                           void* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int64_t base = (int64_t)row * dim;
    auto value = [&](int j) {
        const float v = load_act<DT>(y, base + j);
        return GATED ? v * silu_exact(load_act<DT>(z, base + j)) : v;
    };
    // four strided elements per lane per step: four independent loads in flight
    float sum = 0.0f;
    int j0 = lane;
    for (; j0 + 3 * kWave < dim; j0 += 4 * kWave) {
        float g[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) g[u] = value(j0 + u * kWave);
#pragma unroll
        for (int u = 0; u < 4; ++u) sum = __fmaf_rn(g[u], g[u], sum);
    }
    for (; j0 < dim; j0 += kWave) {
        const float g = value(j0);
        sum = __fmaf_rn(g, g, sum);
    }
    sum = wave_sum(sum);
    const float inv = 1.0f / sqrtf(sum / static_cast<float>(dim) + eps);
    j0 = lane;
    for (; j0 + 3 * kWave < dim; j0 += 4 * kWave) {
        float o[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) o[u] = value(j0 + u * kWave) * inv;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (gamma) o[u] = o[u] * gamma[j0 + u * kWave];
            store_act<ODT>(out, base + j0 + u * kWave, o[u]);
        }
    }
    for (; j0 < dim; j0 += kWave) {
        float o = value(j0) * inv;
        if (gamma) o = o * gamma[j0];
        store_act<ODT>(out, base + j0, o);
    }
}

// ===========================================================================
// The same norm with the row in registers: dim = 512 CH (CH <= 8), each lane
// holding 8 consecutive elements per 512-element chunk, loaded with 16-byte
// loads in one round (a decode row pays one memory latency per tensor instead
// of one per four strided elements).  Rows 16-byte aligned.
// ===========================================================================
template <int DT>
__device__ __forceinline__ void load8v(const void* p, int64_t i, float v[8]) {
    if constexpr (DT == NSOSX_F32) {
        const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
        const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
        const uint4 a = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + i);
        const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            v[2 * k] = __uint_as_float(w[k] << 16);
            v[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
        }
    }
}

template <int ODT>
__device__ __forceinline__ void store8v(void* p, int64_t i, const float v[8]) {
    if constexpr (ODT == NSOSX_F32) {
        float* o = static_cast<float*>(p) + i;
        *reinterpret_cast<float4*>(o) = make_float4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<float4*>(o + 4) = make_float4(v[4], v[5], v[6], v[7]);
    } else {
        *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p) + i) =
            make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                       pack_bf16x2(v[6], v[7]));
    }
}

// QUANT: the next BitLinear's int8 input quantization of the normed row (as stored in
// ODT) in the same pass: absmax, act_scale and codes (ties to even; dim % 8 == 0 here),
// and out only when non-null.
template <int DT, int ODT, bool GATED, int CH, bool QUANT = false>
__global__ __launch_bounds__(256) void rmsnorm_rows_reg_kernel(const void* __restrict__ y,
                                                               const void* __restrict__ z,
                                                               const float* __restrict__ gamma,
                                                               int rows, float eps,
                                                               void* __restrict__ out,
                                                               int8_t* __restrict__ q = nullptr,
                                                               float* __restrict__ act_scale = nullptr,
                                                               float q_max = 0.0f) {
    constexpr int dim = 512 * CH;
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int64_t base = (int64_t)row * dim;
    float g[CH][8];
#pragma unroll
    for (int c = 0; c < CH; ++c) load8v<DT>(y, base + (c * 64 + lane) * 8, g[c]);
    // gamma is fetched with the row, so the output pass waits on no further load
    float gm[CH][8];
    if (gamma) {
#pragma unroll
        for (int c = 0; c < CH; ++c) load8v<NSOSX_F32>(gamma, (c * 64 + lane) * 8, gm[c]);
    }
    if (GATED) {
        float zv[CH][8];
#pragma unroll
        for (int c = 0; c < CH; ++c) load8v<DT>(z, base + (c * 64 + lane) * 8, zv[c]);
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int k = 0; k < 8; ++k) g[c][k] = g[c][k] * silu_exact(zv[c][k]);
    }
    float sum = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int k = 0; k < 8; ++k) sum = __fmaf_rn(g[c][k], g[c][k], sum);
    sum = wave_sum(sum);
    const float inv = 1.0f / sqrtf(sum / static_cast<float>(dim) + eps);
    float mx = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int e0 = (c * 64 + lane) * 8;
        float o[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            o[k] = g[c][k] * inv;
            if (gamma) o[k] = o[k] * gm[c][k];
        }
        if (!QUANT || out) store8v<ODT>(out, base + e0, o);
        if constexpr (QUANT) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                g[c][k] = round_act<ODT>(o[k]);  // the value as stored, kept for the codes
                mx = fmaxf(mx, fabsf(g[c][k]));
            }
        }
    }
    if constexpr (QUANT) {
        mx = wave_max(mx);
        const float denom = __fadd_rn(mx, 1e-8f);
        const float sc = __fdiv_rn(q_max, denom);
        if (lane == 0) act_scale[row] = __fdiv_rn(denom, q_max);
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            float code[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) code[k] = clamp127(rintf(__fmul_rn(g[c][k], sc)));
            *reinterpret_cast<uint2*>(q + base + (c * 64 + lane) * 8) =
                make_uint2(pack4_i8(code[0], code[1], code[2], code[3]),
                           pack4_i8(code[4], code[5], code[6], code[7]));
        }
    }
}

// ===========================================================================
// residual = x + delta (stored in the activation dtype); when norm_out is
// given, norm_out = rmsnorm(residual as stored) [* gamma].  One wave per row.
// ===========================================================================
template <int DT>
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(const void* __restrict__ x,
                                                          const void* __restrict__ delta,
                                                          const float* __restrict__ gamma,
                                                          int rows, int dim, float eps,
                                                          void* __restrict__ residual,
                                                          void* __restrict__ norm_out) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int64_t base = (int64_t)row * dim;
    float sum = 0.0f;
    for (int j = lane; j < dim; j += kWave) {
        store_act<DT>(residual, base + j,
                      load_act<DT>(x, base + j) + load_act<DT>(delta, base + j));
    }
    if (!norm_out) return;
    // each lane re-reads only what it wrote itself: no cross-lane ordering needed
    for (int j = lane; j < dim; j += kWave) {
        const float r = load_act<DT>(residual, base + j);
        sum = __fmaf_rn(r, r, sum);
    }
    sum = wave_sum(sum);
    const float inv = 1.0f / sqrtf(sum / static_cast<float>(dim) + eps);
    for (int j = lane; j < dim; j += kWave) {
        float o = load_act<DT>(residual, base + j) * inv;
        if (gamma) o = o * gamma[j];
        store_act<DT>(norm_out, base + j, o);
    }
}

// ===========================================================================
// Decode conv ring: per (row, channel) value = bias; value += w[j] * src_j for
// j < W, src_j = ring[row][j][c] for j < W - 1 and the new input for the last
// tap; out = silu(value) (or value); the ring shifts one slot and takes the
// new input.  ring: f32 [rows, W-1, C].  Thread = (row, channel).
// ===========================================================================
template <int DT, int ODT>
__global__ __launch_bounds__(256) void conv_step_kernel(const void* __restrict__ x,
                                                        int64_t x_stride, int rows, int C,
                                                        const float* __restrict__ w,
                                                        const float* __restrict__ bias, int W,
                                                        float* __restrict__ ring, int silu,
                                                        void* __restrict__ out) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    const int r = blockIdx.y;
    if (c >= C || r >= rows) return;
    const int taps = W - 1;
    float* rg = ring + (int64_t)r * taps * C + c;
    const float cur = load_act<DT>(x, (int64_t)r * x_stride + c);
    float v = bias ? bias[c] : 0.0f;
    for (int j = 0; j < W; ++j) {
        const float src = j < taps ? rg[(int64_t)j * C] : cur;
        v = __fmaf_rn(w[(int64_t)c * W + j], src, v);
    }
    store_act<ODT>(out, (int64_t)r * C + c, silu ? silu_exact(v) : v);
    for (int s = 0; s + 1 < taps; ++s) rg[(int64_t)s * C] = rg[(int64_t)(s + 1) * C];
    if (taps > 0) rg[(int64_t)(taps - 1) * C] = cur;
}

}  // namespace nsosx

using namespace nsosx;

extern "C" int nsosx_rmsnorm_gated(const void* y, const void* z, const float* gamma, int rows,
                                   int dim, float eps, int act_dtype, void* out, int out_dtype,
                                   void* stream) {
    if (!y || !out) return fail(NSOSX_ERR_INVALID, "rmsnorm_gated: null pointer");
    if (rows < 0 || dim <= 0 || !(eps > 0.0f) || !std::isfinite(eps))
        return fail(NSOSX_ERR_INVALID, "rmsnorm_gated: need rows >= 0, dim > 0, finite eps > 0");
    if (!valid_dtype(act_dtype) || !valid_dtype(out_dtype))
        return fail(NSOSX_ERR_INVALID, "rmsnorm_gated: bad dtype");
    if (rows == 0) return NSOSX_OK;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid((rows + 3) / 4), block(256);
    const bool reg = dim % 512 == 0 && dim <= 4096 &&
                     ((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(z) |
                       reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(gamma)) & 15) == 0;
    if (reg) {
#define NSOSX_RNR(D, O, GT, CH)                                                                  \
    hipLaunchKernelGGL((rmsnorm_rows_reg_kernel<D, O, GT, CH>), grid, block, 0, st, y, z, gamma, \
                       rows, eps, out);
#define NSOSX_RNR_CH(D, O, GT)                                \
    switch (dim / 512) {                                      \
        case 1: NSOSX_RNR(D, O, GT, 1) break;                 \
        case 2: NSOSX_RNR(D, O, GT, 2) break;                 \
        case 3: NSOSX_RNR(D, O, GT, 3) break;                 \
        case 4: NSOSX_RNR(D, O, GT, 4) break;                 \
        case 5: NSOSX_RNR(D, O, GT, 5) break;                 \
        case 6: NSOSX_RNR(D, O, GT, 6) break;                 \
        case 7: NSOSX_RNR(D, O, GT, 7) break;                 \
        default: NSOSX_RNR(D, O, GT, 8) break;                \
    }
#define NSOSX_RNR_G(D, O) \
    if (z) { NSOSX_RNR_CH(D, O, true) } else { NSOSX_RNR_CH(D, O, false) }
        if (act_dtype == NSOSX_F32) {
            if (out_dtype == NSOSX_F32) { NSOSX_RNR_G(NSOSX_F32, NSOSX_F32) } else { NSOSX_RNR_G(NSOSX_F32, NSOSX_BF16) }
        } else {
            if (out_dtype == NSOSX_F32) { NSOSX_RNR_G(NSOSX_BF16, NSOSX_F32) } else { NSOSX_RNR_G(NSOSX_BF16, NSOSX_BF16) }
        }
#undef NSOSX_RNR_G
#undef NSOSX_RNR_CH
#undef NSOSX_RNR
        return check_launch("rmsnorm_gated");
    }
#define NSOSX_RN(D, O)                                                                          \
    if (z) hipLaunchKernelGGL((rmsnorm_rows_kernel<D, O, true>), grid, block, 0, st, y, z,       \
                              gamma, rows, dim, eps, out);                                       \
    else hipLaunchKernelGGL((rmsnorm_rows_kernel<D, O, false>), grid, block, 0, st, y, z, gamma, \
                            rows, dim, eps, out);
    if (act_dtype == NSOSX_F32) {
        if (out_dtype == NSOSX_F32) { NSOSX_RN(NSOSX_F32, NSOSX_F32) } else { NSOSX_RN(NSOSX_F32, NSOSX_BF16) }
    } else {
        if (out_dtype == NSOSX_F32) { NSOSX_RN(NSOSX_BF16, NSOSX_F32) } else { NSOSX_RN(NSOSX_BF16, NSOSX_BF16) }
    }
#undef NSOSX_RN
    return check_launch("rmsnorm_gated");
}

extern "C" int nsosx_rmsnorm_gated_quant(const void* y, const void* z, const float* gamma,
                                         int rows, int dim, float eps, int act_dtype, void* out,
                                         int out_dtype, int bits, int8_t* q, float* act_scale,
                                         void* stream) {
    if (!y || !q || !act_scale) return fail(NSOSX_ERR_INVALID, "rmsnorm_gated_quant: null pointer");
    if (rows < 0 || dim <= 0 || !(eps > 0.0f) || !std::isfinite(eps))
        return fail(NSOSX_ERR_INVALID,
                    "rmsnorm_gated_quant: need rows >= 0, dim > 0, finite eps > 0");
    if (!valid_dtype(act_dtype) || !valid_dtype(out_dtype))
        return fail(NSOSX_ERR_INVALID, "rmsnorm_gated_quant: bad dtype");
    if (bits < 2 || bits > 8)
        return fail(NSOSX_ERR_INVALID, "rmsnorm_gated_quant: bits must be in [2, 8]");
    if (rows == 0) return NSOSX_OK;
    const bool reg = dim % 512 == 0 && dim <= 4096 &&
                     ((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(z) |
                       reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(gamma) |
                       reinterpret_cast<uintptr_t>(q)) & 15) == 0;
    if (!reg) {
        // the two-pass form: the normed rows are the quantization's input
        if (!out)
            return fail(NSOSX_ERR_INVALID,
                        "rmsnorm_gated_quant: out is required unless dim % 512 == 0, dim <= 4096 "
                        "and the buffers are 16-byte aligned");
        int rc = nsosx_rmsnorm_gated(y, z, gamma, rows, dim, eps, act_dtype, out, out_dtype, stream);
        if (rc) return rc;
        return nsosx_quantize_act_i8(out, out_dtype, rows, dim, bits, 0, q, act_scale, nullptr,
                                     stream);
    }
    const float qm = bits <= 2 ? 1.0f : static_cast<float>((1 << (bits - 1)) - 1);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid((rows + 3) / 4), block(256);
#define NSOSX_RNQ(D, O, GT, CH)                                                                  \
    hipLaunchKernelGGL((rmsnorm_rows_reg_kernel<D, O, GT, CH, true>), grid, block, 0, st, y, z,  \
                       gamma, rows, eps, out, q, act_scale, qm);
#define NSOSX_RNQ_CH(D, O, GT)                                \
    switch (dim / 512) {                                      \
        case 1: NSOSX_RNQ(D, O, GT, 1) break;                 \
        case 2: NSOSX_RNQ(D, O, GT, 2) break;                 \
        case 3: NSOSX_RNQ(D, O, GT, 3) break;                 \
        case 4: NSOSX_RNQ(D, O, GT, 4) break;                 \
        case 5: NSOSX_RNQ(D, O, GT, 5) break;                 \
        case 6: NSOSX_RNQ(D, O, GT, 6) break;                 \
        case 7: NSOSX_RNQ(D, O, GT, 7) break;                 \
        default: NSOSX_RNQ(D, O, GT, 8) break;                \
    }
#define NSOSX_RNQ_G(D, O) \
    if (z) { NSOSX_RNQ_CH(D, O, true) } else { NSOSX_RNQ_CH(D, O, false) }
    if (act_dtype == NSOSX_F32) {
        if (out_dtype == NSOSX_F32) { NSOSX_RNQ_G(NSOSX_F32, NSOSX_F32) } else { NSOSX_RNQ_G(NSOSX_F32, NSOSX_BF16) }
    } else {
        if (out_dtype == NSOSX_F32) { NSOSX_RNQ_G(NSOSX_BF16, NSOSX_F32) } else { NSOSX_RNQ_G(NSOSX_BF16, NSOSX_BF16) }
    }
#undef NSOSX_RNQ_G
#undef NSOSX_RNQ_CH
#undef NSOSX_RNQ
    return check_launch("rmsnorm_gated_quant");
}

extern "C" int nsosx_add_rmsnorm(const void* x, const void* delta, const float* gamma, int rows,
                                 int dim, float eps, int act_dtype, void* residual_out,
                                 void* norm_out, void* stream) {
    if (!x || !delta || !residual_out) return fail(NSOSX_ERR_INVALID, "add_rmsnorm: null pointer");
    if (rows < 0 || dim <= 0 || (norm_out && (!(eps > 0.0f) || !std::isfinite(eps))))
        return fail(NSOSX_ERR_INVALID, "add_rmsnorm: need rows >= 0, dim > 0, finite eps > 0");
    if (!valid_dtype(act_dtype)) return fail(NSOSX_ERR_INVALID, "add_rmsnorm: bad dtype");
    if (rows == 0) return NSOSX_OK;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid((rows + 3) / 4), block(256);
    if (act_dtype == NSOSX_F32)
        hipLaunchKernelGGL((add_rmsnorm_kernel<NSOSX_F32>), grid, block, 0, st, x, delta, gamma,
                           rows, dim, eps, residual_out, norm_out);
    else
        hipLaunchKernelGGL((add_rmsnorm_kernel<NSOSX_BF16>), grid, block, 0, st, x, delta, gamma,
                           rows, dim, eps, residual_out, norm_out);
    return check_launch("add_rmsnorm");
}

extern "C" int nsosx_conv_step(const void* x, int x_dtype, int64_t x_stride, int rows,
                               int channels, const float* weight, const float* bias, int width,
                               float* ring, int apply_silu, void* out, int out_dtype,
                               void* stream) {
    if (!x || !weight || !out || (width > 1 && !ring))
        return fail(NSOSX_ERR_INVALID, "conv_step: null pointer");
    if (rows < 0 || rows > 65535 || channels <= 0 || width <= 0 || width > 64 ||
        x_stride < channels)
        return fail(NSOSX_ERR_INVALID, "conv_step: bad shape");
    if (!valid_dtype(x_dtype) || !valid_dtype(out_dtype))
        return fail(NSOSX_ERR_INVALID, "conv_step: bad dtype");
    if (rows == 0) return NSOSX_OK;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid((channels + 255) / 256, rows), block(256);
#define NSOSX_CS(I, O)                                                                         \
    hipLaunchKernelGGL((conv_step_kernel<I, O>), grid, block, 0, st, x, x_stride, rows, channels, \
                       weight, bias, width, ring, apply_silu, out);
    if (x_dtype == NSOSX_F32) {
        if (out_dtype == NSOSX_F32) { NSOSX_CS(NSOSX_F32, NSOSX_F32) } else { NSOSX_CS(NSOSX_F32, NSOSX_BF16) }
    } else {
        if (out_dtype == NSOSX_F32) { NSOSX_CS(NSOSX_BF16, NSOSX_F32) } else { NSOSX_CS(NSOSX_BF16, NSOSX_BF16) }
    }
#undef NSOSX_CS
    return check_launch("conv_step");
}
