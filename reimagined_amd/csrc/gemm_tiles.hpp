// Device code of the ternary MFMA GEMMs (the block tiles, their LDS stages and
// epilogues, the XCD-aware tile order and the grouped launch's tile walk), shared
// by the dense GEMMs (gemm.hip) and the grouped expert GEMMs (gemm_grouped.hip,
// gemm_grouped_mfma.hip).
//
// Reference semantics (OXN/nsos/ of vitorGgC569/reimagined):
//   GEMM + affine src/bitnet_adapter_avx2.cpp:52-158
//   packed format src/bitnet_adapter.cpp:570-606
#pragma once
#include "bitlinear.hpp"

namespace nsosx {

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

constexpr int kBN = 256, kBM = 128, kBK = 64;
constexpr int kXStride = 80;  // bytes per activation row in LDS


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

// A tile's int32 accumulators as raw partial sums: int4 j (0..31) of thread t, its
// acc[j / 16][(j / 4) % 4][4 (j % 4) .. + 3], at (j * 256 + t) * 4 (consecutive threads,
// consecutive 16 bytes).  32768 ints per tile.
constexpr int kG3TileInts = kG3BN * kG3BM;

__device__ __forceinline__ void gemm3_store_raw(const v16i (&acc)[2][4], int32_t* __restrict__ raw) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int j = (a * 4 + b) * 4 + c;
                *reinterpret_cast<int4*>(raw + (j * kGemm3Threads + tid) * 4) =
                    make_int4(acc[a][b][4 * c], acc[a][b][4 * c + 1], acc[a][b][4 * c + 2],
                              acc[a][b][4 * c + 3]);
            }
}

template <int YDT, bool ACC_OUT, bool GATHER, bool SQRELU>
__device__ __forceinline__ void gemm3_store(const GemmProblem& pb, const float* __restrict__ act_scale,
                                            const int32_t* __restrict__ perm, int seg_begin,
                                            int seg_rows, int n0, int m0, void* y,
                                            int32_t* acc_out, const v16i (&acc)[2][4], char* smem);

// MB: 32-row blocks of the tile that hold rows (a partial last tile of an expert's
// segment skips the loads and MFMAs of its empty blocks; their accumulators stay zero
// and their rows are never stored).  k stages [kt0, kt1) (kt1 < 0: to the end); with
// `raw` the tile's partial int32 sums are written there (gemm3_store_raw, before the
// MFMA layout's shift) instead of the epilogue.
template <int YDT, bool ACC_OUT, bool GATHER, bool SQRELU, bool SWZ = false, int MB = 4>
__device__ __forceinline__ void gemm3_tile(const GemmProblem& pb, const int8_t* __restrict__ q,
                                           const float* __restrict__ act_scale,
                                           const int32_t* __restrict__ perm, int seg_begin,
                                           int seg_rows, int n0, int m0, void* y,
                                           int32_t* acc_out, char* smem, int kt0 = 0,
                                           int kt1 = -1, int32_t* raw = nullptr) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;        // wave = 64-row slice of n
    const int W16 = pb.K >> 4;
    const int KT = kt1 < 0 ? pb.K / kG3BK : kt1;

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

    fetch(kt0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    put(kt0);
    if (kt0 + 1 < KT) fetch(kt0 + 1);
    for (int kt = kt0; kt < KT; ++kt) {
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
    if (raw) {
        gemm3_store_raw(acc, raw);
        return;
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
    gemm3_store<YDT, ACC_OUT, GATHER, SQRELU>(pb, act_scale, perm, seg_begin, seg_rows, n0, m0, y,
                                              acc_out, acc, smem);
}

// The epilogue of a 256 x 128 tile from its int32 sums: whole-row-segment bf16 / f32
// stores through the idle stage ring where the tile lies inside N and the pointers
// allow, else gemm3_epilogue.
template <int YDT, bool ACC_OUT, bool GATHER, bool SQRELU>
__device__ __forceinline__ void gemm3_store(const GemmProblem& pb, const float* __restrict__ act_scale,
                                            const int32_t* __restrict__ perm, int seg_begin,
                                            int seg_rows, int n0, int m0, void* y,
                                            int32_t* acc_out, const v16i (&acc)[2][4], char* smem) {
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
                                                int seg_rows, int n0, int m0, void* y, char* smem,
                                                int kt0 = 0, int kt1 = -1,
                                                int32_t* raw = nullptr) {
    const int rows = seg_rows - m0;
    if (rows > 96)
        gemm3_tile<YDT, false, GATHER, SQRELU, SWZ, 4>(pb, q, act_scale, perm, seg_begin, seg_rows,
                                                        n0, m0, y, nullptr, smem, kt0, kt1, raw);
    else if (rows > 64)
        gemm3_tile<YDT, false, GATHER, SQRELU, SWZ, 3>(pb, q, act_scale, perm, seg_begin, seg_rows,
                                                        n0, m0, y, nullptr, smem, kt0, kt1, raw);
    else if (rows > 32)
        gemm3_tile<YDT, false, GATHER, SQRELU, SWZ, 2>(pb, q, act_scale, perm, seg_begin, seg_rows,
                                                        n0, m0, y, nullptr, smem, kt0, kt1, raw);
    else
        gemm3_tile<YDT, false, GATHER, SQRELU, SWZ, 1>(pb, q, act_scale, perm, seg_begin, seg_rows,
                                                        n0, m0, y, nullptr, smem, kt0, kt1, raw);
}

}  // namespace nsosx
