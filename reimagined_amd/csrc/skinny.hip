// BitLinear decode GEMV for small token batches (2 <= M <= 32) on gfx950's
// v_mfma_i32_16x16x64_i8, and its grouped form.
//
// Reference semantics (OXN/nsos/ of vitorGgC569/reimagined):
//   GEMM + affine src/bitnet_adapter_avx2.cpp:52-158
//   packed format src/bitnet_adapter.cpp:570-606
#include "bitlinear.hpp"

namespace nsosx {

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
bool skinny_ok(int M, int K, int N) {
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
// 4 x 4 transpose of one dword per lane across the four 16-lane rows: lane row g
// holds slots u = 0..3 (x, y, z, w), and comes out holding slot g of rows u = 0..3.
__device__ __forceinline__ void transpose_rows4(uint32_t (&v)[4]) {
    const auto p02 = __builtin_amdgcn_permlane32_swap(v[0], v[2], false, false);
    const auto p13 = __builtin_amdgcn_permlane32_swap(v[1], v[3], false, false);
    const auto p01 = __builtin_amdgcn_permlane16_swap(p02[0], p13[0], false, false);
    const auto p23 = __builtin_amdgcn_permlane16_swap(p02[1], p13[1], false, false);
    v[0] = p01[0]; v[1] = p01[1]; v[2] = p23[0]; v[3] = p23[1];
}

// RUN: tiles a wave takes back to back.  RUN = 1: tile ti of a wave is wave_id + ti *
// num_waves, two per output batch.  RUN = 4 (N % 16 == 0 and at least one run per wave):
// runs of 4 consecutive tiles (run i of a wave is wave_id + i * num_waves), one output
// batch per run; the run's outputs are transposed across the four 16-lane rows so that
// lane (g, li) holds tile g's 16 outputs of token li, and the four lanes of a token
// store one whole 128-byte line of its bf16 output row (two lines for f32) where the
// strided order stores 32-byte pieces of 16 rows (bf16: regrouped so that each store
// instruction covers 64 contiguous bytes of the row).  RUN = 2 (two m tiles, bf16 out,
// N % 32 == 0): pairs of consecutive tiles in the two-tile batch's registers, the four
// lanes of a token storing its 64 contiguous bytes with one instruction.
template <int MT, int LT, int YDT, bool ACC_OUT, bool SQRELU, bool VEC4, bool ML = false,
          int RUN = 1>
__device__ __forceinline__ void skinny_body(const GemvProblem& pb, const int8_t* __restrict__ q,
                                            const float* __restrict__ act_scale, int M, void* y,
                                            int32_t* acc_out, int wave_id, int num_waves,
                                            char* lds) {
    static_assert(RUN == 1 || (RUN % 4 == 0 && VEC4) ||
                      (RUN == 2 && VEC4 && YDT == NSOSX_BF16 && !ACC_OUT),
                  "runs of tiles need whole 16-output tiles");
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
    const int runs = (tiles + RUN - 1) / RUN;
    if (wave_id >= runs) return;
    const int my_tiles = ((runs - 1 - wave_id) / num_waves + 1) * RUN;
    // the wave's ti-th tile (runs of RUN consecutive tiles, RUN = 1: strided tiles)
    auto tile_of = [&](int ti) { return (wave_id + (ti / RUN) * num_waves) * RUN + ti % RUN; };
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
        const int tile = min(tile_of(min(ti, my_tiles - 1)), tiles - 1);
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
    auto tile_n0 = [&](int ti) { return tile_of(ti) * 16 + 4 * g; };
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
    constexpr int kSkBatch = RUN == 1 ? 2 : RUN;
    // bf16 outputs of a run are kept as packed pairs (outputs 4 g + {0, 1}, 4 g + {2, 3})
    constexpr bool kPack = RUN > 1 && YDT == NSOSX_BF16;
    for (int t0 = 0; t0 < my_tiles; t0 += kSkBatch) {
        float vb[kSkBatch][MT][4];
        int ab[kSkBatch][MT][4];
        uint32_t pk[kSkBatch][MT][2];
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
                if constexpr (kPack) {
                    pk[u][mt][0] = pack_bf16x2(vb[u][mt][0], vb[u][mt][1]);
                    pk[u][mt][1] = pack_bf16x2(vb[u][mt][2], vb[u][mt][3]);
                }
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                mg_cur[r] = mg_nxt[r];
                bs_cur[r] = bs_nxt[r];
            }
        }
        if constexpr (RUN == 2) {
            // a pair of consecutive tiles: row g of the lane rows holds outputs 4 g .. 4 g + 3
            // of both (two packed dwords each); a permlane32 then a permlane16 swap give row g
            // outputs 8 (g & 1) .. + 7 of tile g >> 1, so the four lanes of a token store
            // its 64 contiguous bytes with one instruction (non-temporal)
            const int run0 = tile_of(t0);
            const int ti = t0 + (g >> 1);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int m = mt * 16 + li;
                uint32_t a[2] = {pk[0][mt][0], pk[0][mt][1]}, b[2] = {pk[1][mt][0], pk[1][mt][1]};
#pragma unroll
                for (int d = 0; d < 2; ++d) {
                    const auto p = __builtin_amdgcn_permlane32_swap(a[d], b[d], false, false);
                    const auto s = __builtin_amdgcn_permlane16_swap(p[0], p[1], false, false);
                    a[d] = s[0];
                    b[d] = s[1];
                }
                const bool ok = ti < my_tiles && run0 + (g >> 1) < tiles && m < M;
                const uint32_t e = static_cast<uint32_t>(m * pb.N + (run0 + (g >> 1)) * 16 + 8 * (g & 1));
                __builtin_amdgcn_raw_buffer_store_b128(v4i{(int)a[0], (int)a[1], (int)b[0], (int)b[1]},
                                                       ry, ok ? e * 2u : 0x80000000u, 0, 2);
            }
            continue;
        }
        if constexpr (RUN > 1) {
#pragma unroll
            for (int qd = 0; qd < RUN / 4; ++qd) {
            // lane (g, li): tile t0 + 4 qd + g of the run, token mt * 16 + li, all 16 outputs
            const int tile = tile_of(t0 + 4 * qd + g);
            const int n0 = tile * 16;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int m = mt * 16 + li;
                const bool ok = tile < tiles && m < M;
                const uint32_t e = static_cast<uint32_t>(m * pb.N + n0);
                if (ACC_OUT) {
                    uint32_t c[4][4];  // c[r][u]: output 4 u + r of the lane's tile
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
#pragma unroll
                        for (int u = 0; u < 4; ++u)
                            c[r][u] = static_cast<uint32_t>(ab[4 * qd + u][mt][r]);
                        transpose_rows4(c[r]);
                    }
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        __builtin_amdgcn_raw_buffer_store_b128(
                            v4i{(int)c[0][u], (int)c[1][u], (int)c[2][u], (int)c[3][u]}, racc,
                            ok ? (e + 4 * u) * 4u : 0x80000000u, 0, 0);
                }
                if (y) {
                    if constexpr (YDT == NSOSX_F32) {
                        uint32_t c[4][4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
#pragma unroll
                            for (int u = 0; u < 4; ++u)
                                c[r][u] = __float_as_uint(vb[4 * qd + u][mt][r]);
                            transpose_rows4(c[r]);
                        }
#pragma unroll
                        for (int u = 0; u < 4; ++u)
                            __builtin_amdgcn_raw_buffer_store_b128(
                                v4i{(int)c[0][u], (int)c[1][u], (int)c[2][u], (int)c[3][u]}, ry,
                                ok ? (e + 4 * u) * 4u : 0x80000000u, 0, 0);
                    } else {
                        uint32_t lo[4], hi[4];  // outputs 4 u + {0, 1} and 4 u + {2, 3}
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            lo[u] = pk[4 * qd + u][mt][0];
                            hi[u] = pk[4 * qd + u][mt][1];
                        }
                        transpose_rows4(lo);
                        transpose_rows4(hi);
                        // lane row g now holds tile g of the run: halves A (outputs 0-7) and
                        // B (8-15); two more swaps give row g half g & 1 of tile g >> 1 (in A)
                        // and of tile 2 + (g >> 1) (in B), so each store covers 64 contiguous
                        // bytes of the token's row
                        uint32_t A[4] = {lo[0], hi[0], lo[1], hi[1]};
                        uint32_t Bh[4] = {lo[2], hi[2], lo[3], hi[3]};
#pragma unroll
                        for (int d = 0; d < 4; ++d) {
                            const auto p = __builtin_amdgcn_permlane16_swap(A[d], Bh[d], false, false);
                            A[d] = p[0]; Bh[d] = p[1];
                        }
#pragma unroll
                        for (int d = 0; d < 4; ++d) {
                            const auto p = __builtin_amdgcn_permlane32_swap(A[d], Bh[d], false, false);
                            A[d] = p[0]; Bh[d] = p[1];
                        }
                        const int run0 = tile_of(t0 + 4 * qd);
#pragma unroll
                        for (int h = 0; h < 2; ++h) {
                            const int ti = t0 + 4 * qd + 2 * h + (g >> 1);
                            const bool okh = ti < my_tiles && run0 + 2 * h + (g >> 1) < tiles && m < M;
                            const uint32_t eh = static_cast<uint32_t>(m * pb.N + run0 * 16 + 32 * h + 8 * g);
                            const uint32_t* d4 = h == 0 ? A : Bh;
                            __builtin_amdgcn_raw_buffer_store_b128(
                                v4i{(int)d4[0], (int)d4[1], (int)d4[2], (int)d4[3]},
                                ry, okh ? eh * 2u : 0x80000000u, 0, 2);
                        }
                    }
                }
            }
            }
            continue;
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
    // a selection of -1 (a padding row of the routing) names no view: nothing to do
    const int vi = view_sel ? view_sel[g] : g;
    if (vi < 0) return;
    const nsosx_linear_view v = views[vi];
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
    const int num_waves = gridDim.x * NW;
    // runs of 4 consecutive tiles at 9-16 token rows (one m tile), where every wave gets
    // one: whole-line stores per token row (M = 16 at K = 2048: 0.63 -> 0.66 of HBM; at 8
    // rows or fewer the stores are cheap and the strided order streams the weights
    // better; at two m tiles, or with the int32 sums out, the run's registers spill)
    if (MT == 1 && !ACC_OUT && M > 8 && (pb.N & 15) == 0 && ((pb.N >> 4) + 3) / 4 >= num_waves)
        skinny_body<MT, LT, YDT, ACC_OUT, false, true, ML, MT == 1 ? 4 : 1>(
            pb, q, act_scale, M, y, acc_out, wave_id, num_waves, lds_sk);
    else if (MT == 2 && YDT == NSOSX_BF16 && !ACC_OUT && (pb.N & 31) == 0 &&
             ((pb.N >> 4) + 1) / 2 >= num_waves)
        skinny_body<MT, LT, YDT, ACC_OUT, false, true, ML,
                    (MT == 2 && YDT == NSOSX_BF16 && !ACC_OUT) ? 2 : 1>(
            pb, q, act_scale, M, y, acc_out, wave_id, num_waves, lds_sk);
    else if ((pb.N & 3) == 0)
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

void launch_skinny(const GemvProblem& pb, const int8_t* q, const float* as, int M, void* y,
                   int y_dtype, int32_t* acc, bool mfma_layout, hipStream_t st) {
    if (mfma_layout) {
        if (y_dtype == NSOSX_F32) launch_skinny_t<NSOSX_F32, true>(pb, q, as, M, y, acc, st);
        else launch_skinny_t<NSOSX_BF16, true>(pb, q, as, M, y, acc, st);
    } else {
        if (y_dtype == NSOSX_F32) launch_skinny_t<NSOSX_F32>(pb, q, as, M, y, acc, st);
        else launch_skinny_t<NSOSX_BF16>(pb, q, as, M, y, acc, st);
    }
}

void launch_grouped_skinny(dim3 grid, const nsosx_linear_view* views, const int8_t* q,
                           int64_t q_stride, const float* act_scale, int64_t scale_stride, int M,
                           void* y, int64_t y_stride, int y_dtype, hipStream_t st) {
    if (y_dtype == NSOSX_F32)
        hipLaunchKernelGGL((grouped_skinny_kernel<NSOSX_F32, false>), grid, dim3(256),
                           kGroupedSkinnyLds, st, views, nullptr, q, q_stride, 1, act_scale,
                           scale_stride, M, y, y_stride);
    else
        hipLaunchKernelGGL((grouped_skinny_kernel<NSOSX_BF16, false>), grid, dim3(256),
                           kGroupedSkinnyLds, st, views, nullptr, q, q_stride, 1, act_scale,
                           scale_stride, M, y, y_stride);
}

}  // namespace nsosx
