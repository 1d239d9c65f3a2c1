// The faithful Mamba-2 decode step's shared pieces (the step's two launches in
// scan.hip; the out_proj GEMV that takes the norm as its prologue in
// bitlinear.hip): the argument block and the per-row gated norm + int8
// quantization.
#pragma once

#include "common.hpp"

namespace nsosx {

constexpr int kM2MaxInner = 8192;   // g and gamma of one row in LDS
constexpr int kM2MaxGS = 1024;      // B and C of one row in LDS
constexpr int kM2MaxW = 4;
constexpr int kM2NormThreads = 512;
constexpr int kM2Rounds = kM2MaxInner / (kM2NormThreads * 4);  // 4-element chunks per thread

struct M2StepArgs {
    const void* x;            // [rows, inner]
    const void* z;            // [rows, inner]
    const void* B;            // [rows, GS], row stride bcdt_stride
    const void* C;
    const void* dt;           // [rows, H], row stride bcdt_stride
    int64_t bcdt_stride;
    const float* conv_w;      // [inner + 2 GS, W]
    const float* conv_b;      // [inner + 2 GS] or null
    float* ring;              // [rows, W - 1, inner + 2 GS]
    const float* a_log;       // [H]
    const float* dskip;       // [H]
    const float* norm_w;      // [inner] or null
    float eps;
    float q_max;
    int H, P, N, G, W;
    float* state;             // [rows, inner, N]
    void* y;                  // [rows, inner]
    int8_t* q;                // [rows, inner]
    float* act_scale;         // [rows]
};


// Row r of the step's second half, by one workgroup of NT threads: the B / C ring
// slots shifted (shift_ring: every reader, the scan launch, has finished), g =
// y * SiLU(z) (the gated norm kernel's product) into s_g, the sum of g^2 by one
// wave in the element order of the one-wave-per-row gated norm (lane l: elements
// (c * 64 + l) * 8 + k), inv = 1 / sqrt(mean + eps), normed = g * inv * gamma as
// stored in ADT, its absmax, act_scale (to *scale_out) and the codes (to q_row; ties
// to even over the first inner & ~7 elements, half away from zero after).  ROUNDS
// chunks of 4 elements per thread cover inner (inner <= 4 * NT * ROUNDS).
template <int ADT, int NT, int ROUNDS>
__device__ __forceinline__ void m2_norm_row(const M2StepArgs& a, int r, bool shift_ring,
                                            int8_t* q_row, float* scale_out, float* s_g,
                                            float* s_red, float* s_inv) {
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int inner = a.H * a.P;
    const int GS = a.G * a.N;
    const int CD = inner + 2 * GS;
    const int taps = a.W - 1;
    // every load of the launch first, one memory round trip: y, z and gamma of this
    // thread's chunks (indices past inner re-read the last element), then the B / C
    // ring slots of this thread's channel
    float yv[ROUNDS][4], zv[ROUNDS][4], gm[ROUNDS][4];
    constexpr uintptr_t VA = ADT == NSOSX_F32 ? 15 : 7;  // alignment of a 4-element load
    const bool vec = (inner & 3) == 0 &&
                     ((reinterpret_cast<uintptr_t>(a.y) | reinterpret_cast<uintptr_t>(a.z)) & VA) == 0 &&
                     (reinterpret_cast<uintptr_t>(a.norm_w) & 15) == 0;
    if (vec) {
        // one load per chunk and tensor (chunks past inner re-read the last chunk)
        auto load4 = [&](const void* p, int64_t off, float v[4]) {
            if constexpr (ADT == NSOSX_F32) {
                const float4 t = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + off);
                v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
            } else {
                const uint2 t = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + off);
                v[0] = __uint_as_float(t.x << 16); v[1] = __uint_as_float(t.x & 0xffff0000u);
                v[2] = __uint_as_float(t.y << 16); v[3] = __uint_as_float(t.y & 0xffff0000u);
            }
        };
#pragma unroll
        for (int k = 0; k < ROUNDS; ++k) {
            const int i0 = min((k * NT + tid) * 4, inner - 4);
            load4(a.y, (int64_t)r * inner + i0, yv[k]);
            load4(a.z, (int64_t)r * inner + i0, zv[k]);
            if (a.norm_w) {
                const float4 t = *reinterpret_cast<const float4*>(a.norm_w + i0);
                gm[k][0] = t.x; gm[k][1] = t.y; gm[k][2] = t.z; gm[k][3] = t.w;
            } else {
                gm[k][0] = gm[k][1] = gm[k][2] = gm[k][3] = 1.0f;
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < ROUNDS; ++k)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int idx = min((k * NT + tid) * 4 + e, inner - 1);
                yv[k][e] = load_act<ADT>(a.y, (int64_t)r * inner + idx);
                zv[k][e] = load_act<ADT>(a.z, (int64_t)r * inner + idx);
                gm[k][e] = a.norm_w ? a.norm_w[idx] : 1.0f;
            }
    }
    const int j = tid;  // B / C channel (2 GS <= NT is the common case)
    const bool shift = shift_ring && taps > 0 && j < 2 * GS;
    float* rg = a.ring + (int64_t)r * taps * CD + inner + min(j, 2 * GS - 1);
    float t[kM2MaxW - 1];
    float bcur = 0.0f;
    if (shift) {
        bcur = load_act<ADT>(j < GS ? a.B : a.C, (int64_t)r * a.bcdt_stride + (j < GS ? j : j - GS));
#pragma unroll
        for (int s2 = 0; s2 < kM2MaxW - 1; ++s2) t[s2] = s2 < taps ? rg[(int64_t)s2 * CD] : 0.0f;
    }
    // g = y * SiLU(z), the gated norm kernel's product
#pragma unroll
    for (int k = 0; k < ROUNDS; ++k)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int idx = (k * NT + tid) * 4 + e;
            if (idx < inner) s_g[idx] = yv[k][e] * silu_exact(zv[k][e]);
        }
    // the B / C ring slots: every reader (the scan launch) has finished
    if (shift) {
#pragma unroll
        for (int s2 = 0; s2 + 1 < kM2MaxW - 1; ++s2)
            if (s2 + 1 < taps) rg[(int64_t)s2 * CD] = t[s2 + 1];
        rg[(int64_t)(taps - 1) * CD] = bcur;
    }
    for (int jj = j + NT; shift_ring && taps > 0 && jj < 2 * GS; jj += NT) {
        const float cur2 = load_act<ADT>(jj < GS ? a.B : a.C,
                                         (int64_t)r * a.bcdt_stride + (jj < GS ? jj : jj - GS));
        float* rg2 = a.ring + (int64_t)r * taps * CD + inner + jj;
        float t2[kM2MaxW - 1];
#pragma unroll
        for (int s2 = 0; s2 < kM2MaxW - 1; ++s2) t2[s2] = s2 < taps ? rg2[(int64_t)s2 * CD] : 0.0f;
#pragma unroll
        for (int s2 = 0; s2 + 1 < kM2MaxW - 1; ++s2)
            if (s2 + 1 < taps) rg2[(int64_t)s2 * CD] = t2[s2 + 1];
        rg2[(int64_t)(taps - 1) * CD] = cur2;
    }
    __syncthreads();
    if (wave == 0) {
        // four 512-element chunks per step, their LDS reads issued together; elements
        // past inner (stale LDS) are masked to zero, and fma(0, 0, sum) == sum
        float sum = 0.0f;
        for (int b = 0; b < inner; b += 4 * 8 * kWave) {
            float4 t[4][2];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int e0 = min(b + (u * kWave + lane) * 8, 4 * NT * ROUNDS - 8);
                t[u][0] = *reinterpret_cast<const float4*>(s_g + e0);
                t[u][1] = *reinterpret_cast<const float4*>(s_g + e0 + 4);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float v[8] = {t[u][0].x, t[u][0].y, t[u][0].z, t[u][0].w,
                                    t[u][1].x, t[u][1].y, t[u][1].z, t[u][1].w};
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const float g = b + (u * kWave + lane) * 8 + k < inner ? v[k] : 0.0f;
                    sum = __fmaf_rn(g, g, sum);
                }
            }
        }
        sum = wave_sum(sum);
        if (lane == 0) *s_inv = 1.0f / sqrtf(sum / static_cast<float>(inner) + a.eps);
    }
    __syncthreads();
    const float inv = *s_inv;
    float nv[ROUNDS][4];
    float m = 0.0f;
#pragma unroll
    for (int k = 0; k < ROUNDS; ++k) {
        const int i0 = (k * NT + tid) * 4;
        const float4 t = *reinterpret_cast<const float4*>(s_g + i0);
        const float v[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float o = v[e] * inv;
            if (a.norm_w) o = o * gm[k][e];
            o = i0 + e < inner ? round_act<ADT>(o) : 0.0f;
            nv[k][e] = o;
            m = fmaxf(m, fabsf(o));
        }
    }
    m = wave_max(m);
    if (lane == 0) s_red[wave] = m;
    __syncthreads();
    m = s_red[0];
#pragma unroll
    for (int w = 1; w < NT / kWave; ++w) m = fmaxf(m, s_red[w]);
    const float denom = __fadd_rn(m, 1e-8f);
    const float sc = __fdiv_rn(a.q_max, denom);
    if (tid == 0) *scale_out = __fdiv_rn(denom, a.q_max);
    const int body = inner & ~7;
    int8_t* qr = q_row;
#pragma unroll
    for (int k = 0; k < ROUNDS; ++k) {
        const int i0 = (k * NT + tid) * 4;
        if (i0 >= inner) break;
        float code[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float val = __fmul_rn(nv[k][e], sc);
            code[e] = clamp127(i0 + e < body ? rintf(val) : roundf(val));
        }
        if (i0 + 4 <= inner && ((reinterpret_cast<uintptr_t>(qr) + i0) & 3) == 0) {
            *reinterpret_cast<uint32_t*>(qr + i0) = pack4_i8(code[0], code[1], code[2], code[3]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (i0 + e < inner) qr[i0 + e] = static_cast<int8_t>(static_cast<int>(code[e]));
        }
    }
}

// out_proj GEMV of one decode row with m2_norm_row as its prologue (bitlinear.hip):
// out [1, N] = dequant(codes . packed) with the row's act_scale; N outputs, K = H * P
int launch_mamba2_norm_gemv(const M2StepArgs& a, int act_dtype, const uint32_t* packed,
                            float weight_scale, int N, const float* magnitude, const float* bias,
                            void* out, int out_dtype, hipStream_t st);
// whether launch_mamba2_norm_gemv takes the step: one row, K % 64 == 0, K <= 4096
bool mamba2_norm_gemv_ok(int rows, int K);

}  // namespace nsosx
