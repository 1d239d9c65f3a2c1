// Quantization-aware-training fake-quant kernels (straight-through estimator)
// on gfx950: the device half of the reference's QAT path.
//
// Reference semantics (OXN/nsos/ of vitorGgC569/reimagined):
//   qat_fake_quant_ternary          src/bitnet_gpu_dispatch.cpp:193-217
//                                   (GPU twin fake_quant_ternary_kernel, src/cuda/bitnet_kernels.cu:155-164)
//   qat_fake_quant_ternary_absmean  src/bitnet_gpu_dispatch.cpp:219-245, scale = tensor_abs_mean + 1e-8f
//                                   (tensor_abs_mean: double sum of |w|, src/tensor.cpp:2072-2102)
//   qat_fake_quant_activations      src/bitnet_gpu_dispatch.cpp:247-282 (std::round: half away from zero)
//   qat_ste_clip_weight_grad(_device_scale)  src/bitnet_gpu_dispatch.cpp:284-325
//   their use in the STE backward   src/bitlinear.cpp:1097-1145
//
// Every float operation is the CPU path's own (multiply by the reciprocal of
// scale + 1e-8f, IEEE division), so the outputs are bit-exact with it.  The
// absmean is a double sum in a fixed two-stage order; rounded to float it
// equals the CPU's sequential double sum unless the double total lies within
// about 1e-16 relative of a float rounding boundary.
#include "common.hpp"

#include <cmath>

namespace nsosx {

constexpr int kQatThreads = 256;
constexpr int kQatSumBlocks = 1024;  // stage-1 partial sums of the absmean

__device__ __forceinline__ float ternary_fq(float w, float scale, float inv) {
    const float v = w * inv;
    const float t = v > 0.5f ? 1.0f : (v < -0.5f ? -1.0f : 0.0f);
    return t * scale;
}

// out = ternary(w * inv) * scale with inv = 1 / (scale + 1e-8f); the scale comes
// from `scale_dev` when given (device-resident absmean), else from `scale`.
__global__ __launch_bounds__(kQatThreads) void fake_quant_ternary_kernel(
    const float* __restrict__ w, int64_t n, float scale, const float* __restrict__ scale_dev,
    float* __restrict__ out) {
    const float s = scale_dev ? scale_dev[0] : scale;
    const float inv = 1.0f / (s + 1e-8f);
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        out[i] = ternary_fq(w[i], s, inv);
}

__device__ __forceinline__ double block_sum_f64(double v, double* s_red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) s_red[wave] = v;
    __syncthreads();
    double t = 0.0;
    if (threadIdx.x == 0)
        for (int i = 0; i < kQatThreads / kWave; ++i) t += s_red[i];
    return t;
}

// Stage 1: block b sums |w| over its contiguous slice into partial[b] (double).
__global__ __launch_bounds__(kQatThreads) void abs_sum_partial_kernel(const float* __restrict__ w,
                                                                      int64_t n,
                                                                      double* __restrict__ partial) {
    __shared__ double s_red[kQatThreads / kWave];
    const int64_t per = (n + gridDim.x - 1) / gridDim.x;
    const int64_t lo = blockIdx.x * per;
    const int64_t hi = min(n, lo + per);
    double v = 0.0;
    for (int64_t i = lo + threadIdx.x; i < hi; i += kQatThreads) v += fabs((double)w[i]);
    const double t = block_sum_f64(v, s_red);
    if (threadIdx.x == 0) partial[blockIdx.x] = t;
}

// Stage 2: scale = float(sum / n) + 1e-8f.
__global__ __launch_bounds__(kQatThreads) void abs_mean_finish_kernel(
    const double* __restrict__ partial, int parts, int64_t n, float* __restrict__ scale_out) {
    __shared__ double s_red[kQatThreads / kWave];
    double v = 0.0;
    for (int i = threadIdx.x; i < parts; i += kQatThreads) v += partial[i];
    const double t = block_sum_f64(v, s_red);
    if (threadIdx.x == 0) scale_out[0] = static_cast<float>(t / static_cast<double>(n)) + 1e-8f;
}

// Per-row activation fake-quant: m = max|x|; denom = m + 1e-8f; x * (q_max / denom)
// clamped to +-q_max, rounded half away from zero, times denom / q_max.
__global__ __launch_bounds__(kQatThreads) void fake_quant_activations_kernel(
    const float* __restrict__ x, int K, float q_max, float* __restrict__ out) {
    __shared__ float s_max[kQatThreads / kWave];
    const int64_t base = (int64_t)blockIdx.x * K;
    float m = 0.0f;
    for (int j = threadIdx.x; j < K; j += kQatThreads) m = fmaxf(m, fabsf(x[base + j]));
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) s_max[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
    const float denom = m + 1e-8f;
    const float scale = q_max / denom;
    const float inv_scale = denom / q_max;
    for (int j = threadIdx.x; j < K; j += kQatThreads) {
        const float v = fminf(fmaxf(x[base + j] * scale, -q_max), q_max);
        out[base + j] = roundf(v) * inv_scale;
    }
}

// STE clip: dW = 0 where |w * inv| > 1, inv = 1 / (scale + 1e-8f).
__global__ __launch_bounds__(kQatThreads) void ste_clip_kernel(float* __restrict__ dW,
                                                               const float* __restrict__ w,
                                                               int64_t n, float scale,
                                                               const float* __restrict__ scale_dev) {
    const float s = scale_dev ? scale_dev[0] : scale;
    const float inv = 1.0f / (s + 1e-8f);
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        if (fabsf(w[i] * inv) > 1.0f) dW[i] = 0.0f;
}

static int elementwise_grid(int64_t n) {
    return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>((n + 255) / 256, 4096)));
}

}  // namespace nsosx

using namespace nsosx;

extern "C" int nsosx_qat_fake_quant_ternary(const float* w, int64_t n, float scale, float* out,
                                            void* stream) {
    if (n < 0 || (n > 0 && (!w || !out))) return fail(NSOSX_ERR_INVALID, "qat_fake_quant_ternary: null pointer");
    if (!std::isfinite(scale) || scale <= 0.0f)
        return fail(NSOSX_ERR_INVALID, "qat_fake_quant_ternary requires a finite positive scale");
    if (n == 0) return NSOSX_OK;
    hipLaunchKernelGGL(fake_quant_ternary_kernel, dim3(elementwise_grid(n)), dim3(kQatThreads), 0,
                       static_cast<hipStream_t>(stream), w, n, scale, nullptr, out);
    return check_launch("qat_fake_quant_ternary");
}

extern "C" int64_t nsosx_qat_absmean_workspace(int64_t n) {
    (void)n;
    return static_cast<int64_t>(kQatSumBlocks * sizeof(double));
}

extern "C" int nsosx_qat_fake_quant_ternary_absmean(const float* w, int64_t n, float* out,
                                                    float* scale_out, void* workspace,
                                                    void* stream) {
    if (n < 0) return fail(NSOSX_ERR_INVALID, "qat_fake_quant_ternary_absmean: n < 0");
    if (n == 0) return NSOSX_OK;
    if (!w || !out || !scale_out || !workspace)
        return fail(NSOSX_ERR_INVALID, "qat_fake_quant_ternary_absmean: null pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int parts = static_cast<int>(std::min<int64_t>(kQatSumBlocks, (n + 255) / 256));
    double* partial = static_cast<double*>(workspace);
    hipLaunchKernelGGL(abs_sum_partial_kernel, dim3(parts), dim3(kQatThreads), 0, st, w, n, partial);
    hipLaunchKernelGGL(abs_mean_finish_kernel, dim3(1), dim3(kQatThreads), 0, st, partial, parts, n,
                       scale_out);
    hipLaunchKernelGGL(fake_quant_ternary_kernel, dim3(elementwise_grid(n)), dim3(kQatThreads), 0,
                       st, w, n, 0.0f, scale_out, out);
    return check_launch("qat_fake_quant_ternary_absmean");
}

extern "C" int nsosx_qat_fake_quant_activations(const float* x, int M, int K, int precision_bits,
                                                float* out, void* stream) {
    if (precision_bits < 2 || precision_bits > 8)
        return fail(NSOSX_ERR_INVALID,
                    "qat_fake_quant_activations: precision_bits must be in the closed interval [2, 8]");
    if (M < 0 || K < 0) return fail(NSOSX_ERR_INVALID, "qat_fake_quant_activations: bad shape");
    if (M == 0 || K == 0) return NSOSX_OK;
    if (!x || !out) return fail(NSOSX_ERR_INVALID, "qat_fake_quant_activations: null pointer");
    const float q_max = precision_bits <= 2 ? 1.0f : static_cast<float>((1 << (precision_bits - 1)) - 1);
    hipLaunchKernelGGL(fake_quant_activations_kernel, dim3(M), dim3(kQatThreads), 0,
                       static_cast<hipStream_t>(stream), x, K, q_max, out);
    return check_launch("qat_fake_quant_activations");
}

extern "C" int nsosx_qat_ste_clip_weight_grad(float* dW, const float* w, int64_t n, float scale,
                                              const float* scale_dev, void* stream) {
    if (n < 0 || (n > 0 && (!dW || !w))) return fail(NSOSX_ERR_INVALID, "qat_ste_clip_weight_grad: null pointer");
    if (!scale_dev && (!std::isfinite(scale) || scale <= 0.0f))
        return fail(NSOSX_ERR_INVALID, "qat_ste_clip_weight_grad requires a finite positive scale");
    if (n == 0) return NSOSX_OK;
    hipLaunchKernelGGL(ste_clip_kernel, dim3(elementwise_grid(n)), dim3(kQatThreads), 0,
                       static_cast<hipStream_t>(stream), dW, w, n, scale, scale_dev);
    return check_launch("qat_ste_clip_weight_grad");
}
