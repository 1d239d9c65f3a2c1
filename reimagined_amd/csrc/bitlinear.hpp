// Internal declarations shared by the BitLinear translation units (quant.hip,
// gemv.hip, skinny.hip, gemm.hip, bitlinear.hip): the problem descriptors, the
// device helpers more than one of them uses, and each unit's host launchers.
//
// Reference semantics (OXN/nsos/ of vitorGgC569/reimagined):
//   quantization  src/bitlinear.cpp:240-291, src/bitlinear_quantize_avx2.cpp:65-103
//   RMS_PERI norm src/bitlinear.cpp:460-466, src/tensor.cpp:3455-3492
//   GEMM + affine src/bitnet_adapter_avx2.cpp:52-158
//   packed format src/bitnet_adapter.cpp:570-606
#pragma once
#include "common.hpp"
#include "mamba2_step.hpp"

#include <algorithm>
#include <cmath>

namespace nsosx {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// A ternary GEMV / GEMM problem: packed weights [N, K] (K / 16 words per row) with
// the output affine (weight scale, optional magnitude and bias per output).
struct GemvProblem {
    const uint32_t* packed;
    const float* mag;
    const float* bias;
    float ws;
    int N;
    int K;
};

struct GemmProblem {
    const uint32_t* packed;
    const float* mag;
    const float* bias;
    float ws;
    int N;
    int K;
};

// Block tile of the LDS-staged MFMA GEMMs (n x m x k).
constexpr int kG3BN = 256, kG3BM = 128, kG3BK = 128;

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

// 8 consecutive activations as floats (bf16 widened exactly).
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

// A group of a grouped GEMV with M >= 2 rows that the skinny MFMA body takes:
// K = 1024 or 2048 (its fragments fit the launch's 64 KB of LDS) and whole
// 4-output vectors (N % 4 == 0, 16-byte aligned rows).
__device__ __forceinline__ bool skinny_group(const nsosx_linear_view& v, const void* yb) {
    return (v.inputs == 1024 || v.inputs == 2048) && (v.outputs & 3) == 0 &&
           (reinterpret_cast<uintptr_t>(yb) & 15) == 0;
}

// ---- host launchers (each defined in the unit named) ----------------------
// quant.hip: RMS_PERI (when rms_input) and the int8 codes of x [M, K]
int launch_quantize_dt(const void* x, int dtype, int M, int K, int bits, int rms_input, int8_t* q,
                       float* act_scale, float* rms_ws, hipStream_t st);
// gemv.hip: the VALU GEMV (M <= 8) on the reference words
void launch_gemv(const GemvProblem& pb, const int8_t* q, const float* as, int M, void* y,
                 int y_dtype, int32_t* acc, hipStream_t st);
// skinny.hip: the MFMA decode GEMV (2 <= M <= 32, skinny_ok), on the reference words
// or (mfma_layout) the MFMA-layout words; and the grouped form for nsosx_grouped_gemv
bool skinny_ok(int M, int K, int N);
void launch_skinny(const GemvProblem& pb, const int8_t* q, const float* as, int M, void* y,
                   int y_dtype, int32_t* acc, bool mfma_layout, hipStream_t st);
void launch_grouped_skinny(dim3 grid, const nsosx_linear_view* views, const int8_t* q,
                           int64_t q_stride, const float* act_scale, int64_t scale_stride, int M,
                           void* y, int64_t y_stride, int y_dtype, hipStream_t st);
// gemm.hip: the MFMA GEMMs on the reference words and on the MFMA layout
void launch_gemm(const GemmProblem& pb, const int8_t* q, const float* as, int M, void* y,
                 int y_dtype, int32_t* acc, hipStream_t st);
void launch_gemm_mfma(const GemmProblem& pb, const int8_t* q, const float* as, int M, void* y,
                      int y_dtype, int32_t* acc, hipStream_t st);

}  // namespace nsosx
