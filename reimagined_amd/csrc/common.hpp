// Shared device/host helpers of the nsosx HIP library (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/nsosx.h"

namespace nsosx {

constexpr int kWave = 64;

// ---- error reporting -------------------------------------------------------

void set_error(const std::string& msg);

inline int fail(int status, const std::string& msg) {
    set_error(msg);
    return status;
}

inline int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        return fail(NSOSX_ERR_LAUNCH, std::string(what) + ": " + hipGetErrorString(e));
    }
    return NSOSX_OK;
}

inline bool valid_dtype(int d) { return d == NSOSX_F32 || d == NSOSX_BF16; }

// inv[m] = 1 / sqrt(mean_k x[m,k]^2 + eps), the row scale of Tensor::rmsnorm with its
// in-order sum (bitlinear.hip); x [M, K] in `dtype`.
void launch_rms_inv(const void* x, int dtype, int M, int K, float eps, float* inv,
                    hipStream_t st);

// ---- bf16 <-> f32 -----------------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round to nearest even (v_cvt_pk_bf16_f32); NaN stays a quiet NaN.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const bf16x2_t r = __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t);
    return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

template <int DT>
__device__ __forceinline__ float load_act(const void* p, int64_t i) {
    if constexpr (DT == NSOSX_F32) {
        return static_cast<const float*>(p)[i];
    } else {
        return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
    }
}

// Raw storage word of an activation element: kept unconverted in registers, a
// prefetched value costs no wait until raw_to_f32() is applied where it is used.
template <int DT> struct raw_word { using type = uint32_t; };
template <> struct raw_word<NSOSX_BF16> { using type = uint16_t; };

template <int DT>
__device__ __forceinline__ typename raw_word<DT>::type load_raw(const void* p, int64_t i) {
    using T = typename raw_word<DT>::type;
    return ((const __attribute__((address_space(1))) T*)(p))[i];
}

template <int DT>
__device__ __forceinline__ float raw_to_f32(typename raw_word<DT>::type u) {
    if constexpr (DT == NSOSX_F32) {
        return __uint_as_float(u);
    } else {
        return __uint_as_float(static_cast<uint32_t>(u) << 16);
    }
}

// Raw buffer access (buffer_load / buffer_store with a 32-bit byte offset from a
// resource that carries the base and the extent): a load past the extent
// returns 0 and a store past it is dropped, so running offsets need no clamps.
// Word 3 of the resource (0x00020000) is the untyped 32-bit data format of the
// gfx9 family.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
}

template <int DT>
__device__ __forceinline__ typename raw_word<DT>::type buf_load_raw(__amdgpu_buffer_rsrc_t r,
                                                                    uint32_t byte_off) {
    if constexpr (DT == NSOSX_F32) {
        return __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, 0);
    } else {
        return __builtin_amdgcn_raw_buffer_load_b16(r, byte_off, 0, 0);
    }
}

template <int DT>
__device__ __forceinline__ void buf_store_act(__amdgpu_buffer_rsrc_t r, uint32_t byte_off,
                                              float v) {
    if constexpr (DT == NSOSX_F32) {
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, byte_off, 0, 0);
    } else {
        __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(v), r, byte_off, 0, 0);
    }
}

template <int DT>
__device__ __forceinline__ void store_act(void* p, int64_t i, float v) {
    if constexpr (DT == NSOSX_F32) {
        static_cast<float*>(p)[i] = v;
    } else {
        static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
    }
}

// Value as stored in the activation dtype and read back (bf16: round to nearest even).
template <int DT>
__device__ __forceinline__ float round_act(float v) {
    if constexpr (DT == NSOSX_F32) return v;
    else return bf16_to_f32(f32_to_bf16(v));
}

// ---- activation math ---------------------------------------------------------

// SiLU split on the sign (Tensor::silu, src/tensor.cpp:3261-3282; Mamba2SSD::silu_stable,
// src/mamba2.cpp:737-739): libm expf, IEEE division
__device__ __forceinline__ float silu_exact(float v) {
    const float sig = v >= 0.0f ? 1.0f / (1.0f + expf(-v)) : expf(v) / (1.0f + expf(v));
    return v * sig;
}

// int8 codes: clamp to [-127, 127], four codes packed little-endian
__device__ __forceinline__ float clamp127(float c) { return fminf(fmaxf(c, -127.0f), 127.0f); }

__device__ __forceinline__ uint32_t pack4_i8(float a, float b, float c, float d) {
    const uint32_t ia = static_cast<uint32_t>(static_cast<int>(a)) & 0xffu;
    const uint32_t ib = static_cast<uint32_t>(static_cast<int>(b)) & 0xffu;
    const uint32_t ic = static_cast<uint32_t>(static_cast<int>(c)) & 0xffu;
    const uint32_t id = static_cast<uint32_t>(static_cast<int>(d)) & 0xffu;
    return ia | (ib << 8) | (ic << 16) | (id << 24);
}

// ---- wave reductions (wave64) ---------------------------------------------

// The value of lane (lane ^ O) without a trip through LDS memory: DPP quad
// permutes for 1 and 2, a row rotation by 8 (within a 16-lane row that is lane ^ 8),
// the swizzle unit's xor mode for 4 and 16 (within 32 lanes), and the 32-lane swap
// for 32.  The same exchange as __shfl_xor(v, O), so the butterflies below add and
// compare the same pairs in the same order.
template <int O>
__device__ __forceinline__ float lane_xor(float v) {
    const int u = __float_as_int(v);
    if constexpr (O == 1) {
        return __int_as_float(__builtin_amdgcn_mov_dpp(u, 0xB1, 0xF, 0xF, true));
    } else if constexpr (O == 2) {
        return __int_as_float(__builtin_amdgcn_mov_dpp(u, 0x4E, 0xF, 0xF, true));
    } else if constexpr (O == 8) {
        return __int_as_float(__builtin_amdgcn_mov_dpp(u, 0x128, 0xF, 0xF, true));
    } else if constexpr (O == 4 || O == 16) {
        return __int_as_float(__builtin_amdgcn_ds_swizzle(u, 0x1F | (O << 10)));
    } else {
        static_assert(O == 32, "lane_xor: 1, 2, 4, 8, 16 or 32");
        // lanes 0-31 of the swapped source hold lanes 32-63, lanes 32-63 of the
        // swapped destination lanes 0-31
        const auto p = __builtin_amdgcn_permlane32_swap(static_cast<unsigned>(u),
                                                        static_cast<unsigned>(u), false, false);
        const bool hi = (threadIdx.x & 32) != 0;
        return __uint_as_float(hi ? p[0] : p[1]);
    }
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, lane_xor<32>(v));
    v = fmaxf(v, lane_xor<16>(v));
    v = fmaxf(v, lane_xor<8>(v));
    v = fmaxf(v, lane_xor<4>(v));
    v = fmaxf(v, lane_xor<2>(v));
    v = fmaxf(v, lane_xor<1>(v));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
    v += lane_xor<32>(v);
    v += lane_xor<16>(v);
    v += lane_xor<8>(v);
    v += lane_xor<4>(v);
    v += lane_xor<2>(v);
    v += lane_xor<1>(v);
    return v;
}

__device__ __forceinline__ int wave_sum_i32(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// ---- ternary unpack ----------------------------------------------------------
//
// One packed word holds 16 codes, code j at bits 2j.  unpack_word() returns
// four dwords of int8 values; dword s, byte b holds the value of code 4b+s
// (an order in which every step is a shift, a mask and a byte permute).
// The byte permute looks the 2-bit code up in the table {-1, 0, +1, 0}
// (code 3 is reserved and decodes to 0, as on the reference CPU path).
constexpr uint32_t kTernaryLut = 0x000100FFu;  // bytes: 0xFF, 0x00, 0x01, 0x00

__device__ __forceinline__ void unpack_word(uint32_t p, uint32_t out[4]) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const uint32_t t = (p >> (2 * s)) & 0x03030303u;
        out[s] = __builtin_amdgcn_perm(0u, kTernaryLut, t);
    }
}

// 4x4 byte transpose of 16 activation bytes in natural order (dword d, byte c
// = element 4d+c) into the order unpack_word() produces (dword s, byte b =
// element 4b+s).
__device__ __forceinline__ void transpose16(const uint32_t d[4], uint32_t e[4]) {
    const uint32_t t0 = __builtin_amdgcn_perm(d[1], d[0], 0x05010400u);
    const uint32_t t1 = __builtin_amdgcn_perm(d[1], d[0], 0x07030602u);
    const uint32_t t2 = __builtin_amdgcn_perm(d[3], d[2], 0x05010400u);
    const uint32_t t3 = __builtin_amdgcn_perm(d[3], d[2], 0x07030602u);
    e[0] = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
    e[1] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
    e[2] = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
    e[3] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const u32x4 global_u32x4;
typedef __attribute__((address_space(1))) const uint32_t global_u32;

// 16-byte streaming load that is not expected to be reused (weights of a GEMV).
// The pointer is taken as global memory: a flat load would also count against
// the LDS/scalar wait counter, so every LDS or shuffle wait would drain it.
__device__ __forceinline__ uint4 load_stream16(const uint32_t* p) {
    const u32x4 v = __builtin_nontemporal_load((global_u32x4*)(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}

// ---- dequantizing epilogue (bitnet_adapter_avx2.cpp:36-47,93,150-156) -----
// The reference's apply_output_affine multiplies and adds in separate branches,
// so its build rounds twice (no fma) even under -mfma; so does this.
__device__ __forceinline__ float dequant(int acc, float combined, const float* mag,
                                         const float* bias, int n) {
    float v = __fmul_rn(static_cast<float>(acc), combined);
    if (mag) v = __fmul_rn(v, mag[n]);
    if (bias) v = __fadd_rn(v, bias[n]);
    return v;
}

}  // namespace nsosx
