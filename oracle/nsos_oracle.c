/*
 * nsos_oracle.c -- CPU restatement of the reference hybrid-layer hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see nsos_oracle.h).  Only tests/, the smoke()
 * check of __graft_entry__.py and the cpu_baseline leg of bench.py use it.
 *
 * Rounding contract.  The reference is built by gcc as gnu++20 with
 * -mavx -mfma (OXN/nsos/CMakeLists.txt:19,159), so gcc's default
 * -ffp-contract=fast fuses some multiply-add pairs.  This file is compiled
 * with -ffp-contract=off and spells every fusion the reference's code
 * generation performs as an explicit fmaf(), so the oracle's bits do not
 * depend on this file's compiler flags:
 *   - output affine  value*magnitude, then + bias  -> two roundings: the multiply
 *                    and the add sit in separate branches of apply_output_affine
 *                    (bitnet_adapter_avx2.cpp:36-47), which gcc does not contract
 *   - scan update    decay*state + (delta*B)*x      -> fmaf (mamba2.cpp:2654-2662)
 *   - scan readout   out += state*C                 -> fmaf (mamba2.cpp:2662)
 *   - causal conv    acc += w*in                    -> fmaf (mamba2.cpp:1068-1071)
 *   - RMSNorm        sum_sq += v*v: the -O3 body reduces rounded squares in
 *                    order, the <4-element remainder is fused (tensor.cpp:3480-3484)
 * Those fusion choices are a property of gcc 11.4 with the reference's flags.
 * The output affine, the RMSNorm sum and the BitLinear forward are pinned
 * bit for bit against the reference's own build of those files (oracle/_ref,
 * fixtures in tests/golden/); the scan's are pinned by float64 closed forms.
 */
#include "nsos_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ========================================================================
 * BitLinear weights
 * ====================================================================== */

/* tensor_abs_mean: sum |w| in double, divide in double, round to float.
 * OXN/nsos/src/tensor.cpp:2100-2107 */
float orc_absmean(const float* w, int64_t n) {
    if (n <= 0) return 0.0f;
    double total = 0.0;
    for (int64_t i = 0; i < n; ++i) total += fabs((double)w[i]);
    return (float)(total / (double)n);
}

/* BitLinear::pack_weights: weight_scale = tensor_abs_mean(W) + 1e-8f.
 * OXN/nsos/src/bitlinear.cpp:174 */
float orc_weight_scale(const float* w, int64_t n) {
    return orc_absmean(w, n) + 1e-8f;
}

/* BitLinear::quantize_weights: v = w / (scale + 1e-8f) with
 * scale = absmean + 1e-8f (so 1e-8f is added twice); +1 if v > 0.5,
 * -1 if v < -0.5, else 0.  OXN/nsos/src/bitlinear.cpp:1359-1379 */
void orc_ternary_codes(const float* w, int64_t n, float weight_scale, int8_t* codes) {
    const float denom = weight_scale + 1e-8f;
    for (int64_t i = 0; i < n; ++i) {
        const float v = w[i] / denom;
        codes[i] = v > 0.5f ? 1 : (v < -0.5f ? -1 : 0);
    }
}

/* BitNetAdapter::pack_weights_microsoft_style: 4 codes per byte, element j of
 * each group of four at bits 2j (LSB first), value -1 -> 0, 0 -> 1, +1 -> 2,
 * flat over the row-major [N,K] array, tail byte zero-filled.
 * OXN/nsos/src/bitnet_adapter.cpp:570-588 */
void orc_pack_codes(const int8_t* codes, int64_t n, uint8_t* packed) {
    const int64_t bytes = (n + 3) / 4;
    memset(packed, 0, (size_t)bytes);
    for (int64_t i = 0; i < n; ++i) {
        const uint8_t two = codes[i] < 0 ? 0u : (codes[i] > 0 ? 2u : 1u);
        packed[i >> 2] |= (uint8_t)(two << ((i & 3) * 2));
    }
}

/* unpack_weights_microsoft_style_to_i8 with kDecodeI8Lut {-1,0,+1,0}: the
 * reserved code 3 decodes to 0 on the CPU path.
 * OXN/nsos/src/bitnet_adapter.cpp:31,590-606 */
void orc_unpack_codes(const uint8_t* packed, int64_t n, int8_t* codes) {
    static const int8_t lut[4] = {-1, 0, 1, 0};
    for (int64_t i = 0; i < n; ++i) codes[i] = lut[(packed[i >> 2] >> ((i & 3) * 2)) & 3u];
}

/* Index of the first reserved code 3 (import rejects it), or -1.
 * OXN/nsos/src/bitlinear.cpp:876-885 */
int64_t orc_find_reserved_code(const uint8_t* packed, int64_t n) {
    for (int64_t i = 0; i < n; ++i)
        if (((packed[i >> 2] >> ((i & 3) * 2)) & 3u) == 3u) return i;
    return -1;
}

/* compute_weight_row_sums: exact int32 row sums. OXN/nsos/src/bitlinear.cpp:36-73 */
void orc_row_sums(const int8_t* w, int rows, int cols, int32_t* sums) {
    for (int r = 0; r < rows; ++r) {
        int32_t s = 0;
        for (int c = 0; c < cols; ++c) s += w[(int64_t)r * cols + c];
        sums[r] = s;
    }
}

/* ========================================================================
 * Activations
 * ====================================================================== */

/* q_max = 1 for bits <= 2, else 2^(bits-1) - 1.  OXN/nsos/src/bitlinear.cpp:248-252 */
float orc_q_max(int bits) {
    if (bits <= 2) return 1.0f;
    return (float)(pow(2.0, (double)(bits - 1)) - 1.0);
}

/* Tensor::rmsnorm: per row inv = 1/sqrt(sum_sq/cols + eps), out = x*inv, with
 * the float sum taken in index order.  OXN/nsos/src/tensor.cpp:3455-3492 */
void orc_rmsnorm(const float* x, int rows, int cols, float eps, float* out) {
#pragma omp parallel for
    for (int r = 0; r < rows; ++r) {
        const float* src = x + (int64_t)r * cols;
        float* dst = out + (int64_t)r * cols;
        const int body = cols & ~3;
        float sum_sq = 0.0f;
        for (int j = 0; j < body; ++j) {
            const float sq = src[j] * src[j];
            sum_sq = sum_sq + sq;
        }
        for (int j = body; j < cols; ++j) sum_sq = fmaf(src[j], src[j], sum_sq);
        const float inv = 1.0f / sqrtf(sum_sq / (float)(cols > 1 ? cols : 1) + eps);
        for (int j = 0; j < cols; ++j) dst[j] = src[j] * inv;
    }
}

/* BitLinear::quantize_activations_bitnet on an AVX2 host, followed by the
 * GEMM's int8 cast:
 *   m = max|x| over the row (exact)            bitlinear_quantize_avx2.cpp:65-82
 *   s = q_max / (m + 1e-8f)                     bitlinear.cpp:273
 *   act_scale = (m + 1e-8f) / q_max  (a separate division, not 1/s)   bitlinear.cpp:274
 *   code = round(x*s): ties-to-even for the 8-aligned body
 *          (_mm256_round_ps, bitlinear_quantize_avx2.cpp:89-99), half away
 *          from zero for the K%8 tail (std::round, :100-102)
 *   int8 = clamp(code, -127, 127)               bitnet_adapter_avx2.cpp:95-126 */
void orc_quantize_act(const float* x, int rows, int cols, int bits, int8_t* q,
                      float* act_scale) {
    const float q_max = orc_q_max(bits);
#pragma omp parallel for
    for (int r = 0; r < rows; ++r) {
        const float* src = x + (int64_t)r * cols;
        int8_t* dst = q + (int64_t)r * cols;
        float m = 0.0f;
        for (int j = 0; j < cols; ++j) {
            const float a = fabsf(src[j]);
            if (a > m) m = a;
        }
        const float s = q_max / (m + 1e-8f);
        act_scale[r] = (m + 1e-8f) / q_max;
        const int body = cols & ~7;
        for (int j = 0; j < cols; ++j) {
            const float v = src[j] * s;
            float code = j < body ? nearbyintf(v) : roundf(v);
            if (code > 127.0f) code = 127.0f;
            if (code < -127.0f) code = -127.0f;
            dst[j] = (int8_t)code;
        }
    }
}

/* gemm_158bit_i8 integer core: acc[m,n] = sum_k q[m,k]*w[n,k] (exact int32).
 * OXN/nsos/src/bitnet_adapter_avx2.cpp:128-149 */
void orc_gemm_i8(const int8_t* q, const int8_t* w, int M, int K, int N, int32_t* acc) {
    for (int m = 0; m < M; ++m) {
        const int8_t* a = q + (int64_t)m * K;
        for (int n = 0; n < N; ++n) {
            const int8_t* b = w + (int64_t)n * K;
            int32_t s = 0;
            for (int k = 0; k < K; ++k) s += (int32_t)a[k] * (int32_t)b[k];
            acc[(int64_t)m * N + n] = s;
        }
    }
}

/* Dequantizing epilogue: y = float(acc) * (act_scale*ws), then *magnitude,
 * then +bias, each rounded (the reference build does not fuse them).
 * OXN/nsos/src/bitnet_adapter_avx2.cpp:93,150-156 and apply_output_affine :37-48 */
void orc_dequant(const int32_t* acc, const float* act_scale, float weight_scale,
                 const float* magnitude, const float* bias, int M, int N, float* y) {
    for (int m = 0; m < M; ++m) {
        const float combined = act_scale[m] * weight_scale;
        for (int n = 0; n < N; ++n) {
            float v = (float)acc[(int64_t)m * N + n] * combined;
            if (magnitude) v = v * magnitude[n];
            if (bias) v = v + bias[n];
            y[(int64_t)m * N + n] = v;
        }
    }
}

/* BitLinear::forward on the CPU packed path: optional RMS_PERI norm (eps
 * 1e-6), activation quantization, int8 GEMM, fused output affine.
 * OXN/nsos/src/bitlinear.cpp:439-466 (norm), 690-741 (packed path). */
void orc_bitlinear_forward(const float* x, int M, int K, int N, const uint8_t* packed,
                           float weight_scale, int bits, int rms_input,
                           const float* magnitude, const float* bias, float* y,
                           int8_t* q_out, float* act_scale_out, int32_t* acc_out) {
    float* xn = NULL;
    const float* src = x;
    if (rms_input) {
        xn = (float*)malloc(sizeof(float) * (size_t)M * (size_t)K);
        orc_rmsnorm(x, M, K, 1e-6f, xn);
        src = xn;
    }
    int8_t* q = q_out ? q_out : (int8_t*)malloc((size_t)M * (size_t)K);
    float* as = act_scale_out ? act_scale_out : (float*)malloc(sizeof(float) * (size_t)M);
    int32_t* acc = acc_out ? acc_out : (int32_t*)malloc(sizeof(int32_t) * (size_t)M * (size_t)N);
    int8_t* w = (int8_t*)malloc((size_t)N * (size_t)K);
    orc_unpack_codes(packed, (int64_t)N * K, w);
    orc_quantize_act(src, M, K, bits, q, as);
    orc_gemm_i8(q, w, M, K, N, acc);
    orc_dequant(acc, as, weight_scale, magnitude, bias, M, N, y);
    free(w);
    if (!acc_out) free(acc);
    if (!act_scale_out) free(as);
    if (!q_out) free(q);
    free(xn);
}

/* ========================================================================
 * Elementwise
 * ====================================================================== */

/* Tensor::silu with the sign-split sigmoid. OXN/nsos/src/tensor.cpp:3261-3282 */
float orc_silu(float v) {
    const float sig = v >= 0.0f ? 1.0f / (1.0f + expf(-v)) : expf(v) / (1.0f + expf(v));
    return v * sig;
}

/* Mamba2SSD::softplus_stable. OXN/nsos/src/mamba2.cpp:718-726 */
float orc_softplus(float v) {
    if (v > 20.0f) return v;
    if (v < -20.0f) return expf(v);
    return log1pf(expf(v));
}

/* Tensor::squared_relu: max(x,0)^2. OXN/nsos/src/tensor.cpp:3209-3226 */
void orc_squared_relu(const float* x, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) {
        const float v = x[i] > 0.0f ? x[i] : 0.0f;
        out[i] = v * v;
    }
}

/* ========================================================================
 * Mamba selective scan
 * ====================================================================== */

/* mamba_decay_terms: delta = softplus(dt) in float; decay =
 * exp(-exp(log(delta) + A_log)) in double; log_q > 50 gives 0; a
 * non-finite input gives NaN.  OXN/nsos/src/mamba2.cpp:443-473 */
void orc_decay_terms(float dt_raw, float a_log, float* delta, float* decay) {
    const float d = orc_softplus(dt_raw);
    *delta = d;
    if (!isfinite(dt_raw) || !isfinite(a_log)) {
        *decay = NAN;
        return;
    }
    const double log_delta = dt_raw < -20.0f ? (double)dt_raw : log((double)d);
    const double log_q = log_delta + (double)a_log;
    if (log_q > 50.0) {
        *decay = 0.0f;
        return;
    }
    *decay = (float)exp(-exp(log_q));
}

/* Depthwise causal convolution restarted at every cu_seqlens boundary:
 *   out[t,c] = sum_{j<W} w[c,j] * in[t-(W-1)+j, c]   (zero before the sequence)
 * then + bias[c] and SiLU when requested.
 * OXN/nsos/src/mamba2.cpp:1056-1076 (conv), 2437-2446 (bias, SiLU). */
void orc_conv1d_causal(const float* in, const float* weight, const float* bias,
                       const int32_t* cu_seqlens, int num_seqs, int channels,
                       int width, int apply_silu, float* out) {
    for (int s = 0; s < num_seqs; ++s) {
        const int t0 = cu_seqlens[s];
        const int t1 = cu_seqlens[s + 1];
        for (int t = t0; t < t1; ++t) {
            for (int c = 0; c < channels; ++c) {
                float acc = 0.0f;
                for (int j = 0; j < width; ++j) {
                    const int src_t = t - (width - 1) + j;
                    if (src_t < t0) continue;
                    acc = fmaf(weight[(int64_t)c * width + j],
                               in[(int64_t)src_t * channels + c], acc);
                }
                if (bias) acc = acc + bias[c];
                if (apply_silu) acc = orc_silu(acc);
                out[(int64_t)t * channels + c] = acc;
            }
        }
    }
}

/* Decode conv ring step, CPU streaming path of forward_faithful_step:
 *   v = bias[c]; v += w[c,j] * (j < W-1 ? ring[r][j][c] : x[r,c]) for j < W;
 *   out = silu(v); ring shifts one slot and takes x[r,c].
 * The reference writes `value += w * src` under -mfma, contracted to fma.
 * ring: [rows, W-1, channels].  OXN/nsos/src/mamba2.cpp:4072-4090 */
void orc_conv_step(const float* x, int rows, int channels, const float* weight,
                   const float* bias, int width, float* ring, int apply_silu, float* out) {
    const int taps = width - 1;
    for (int r = 0; r < rows; ++r) {
        float* rg = ring ? ring + (int64_t)r * taps * channels : NULL;
        for (int c = 0; c < channels; ++c) {
            const float cur = x[(int64_t)r * channels + c];
            float v = bias ? bias[c] : 0.0f;
            for (int j = 0; j < width; ++j) {
                const float src = j < taps ? rg[(int64_t)j * channels + c] : cur;
                v = fmaf(weight[(int64_t)c * width + j], src, v);
            }
            out[(int64_t)r * channels + c] = apply_silu ? orc_silu(v) : v;
            for (int s2 = 0; s2 + 1 < taps; ++s2)
                rg[(int64_t)s2 * channels + c] = rg[(int64_t)(s2 + 1) * channels + c];
            if (taps > 0) rg[(int64_t)(taps - 1) * channels + c] = cur;
        }
    }
}

/* Gated RMSNorm epilogue, norm_before_gate = false:
 *   g = y * silu(z)                  Tensor::silu_gate, tensor.cpp:3323-3343
 *   inv = 1 / sqrt(sum g^2 / K + eps), sum in index order
 *                                    Tensor::rmsnorm, tensor.cpp:3455-3492
 *   out = (g * inv) * gamma          Tensor::mul, mamba2.cpp:2677-2680
 * z NULL: plain rmsnorm; gamma NULL: unit weight. */
void orc_rmsnorm_gated(const float* y, const float* z, const float* gamma, int rows, int cols,
                       float eps, float* out) {
    for (int r = 0; r < rows; ++r) {
        const float* yr = y + (int64_t)r * cols;
        const float* zr = z ? z + (int64_t)r * cols : NULL;
        float* dst = out + (int64_t)r * cols;
        for (int j = 0; j < cols; ++j) dst[j] = zr ? yr[j] * orc_silu(zr[j]) : yr[j];
        /* the same sum as orc_rmsnorm: rounded squares added in order, fma tail */
        const int body = cols & ~3;
        float sum_sq = 0.0f;
        for (int j = 0; j < body; ++j) {
            const float sq = dst[j] * dst[j];
            sum_sq = sum_sq + sq;
        }
        for (int j = body; j < cols; ++j) sum_sq = fmaf(dst[j], dst[j], sum_sq);
        const float inv = 1.0f / sqrtf(sum_sq / (float)(cols > 1 ? cols : 1) + eps);
        for (int j = 0; j < cols; ++j) {
            dst[j] = dst[j] * inv;
            if (gamma) dst[j] = dst[j] * gamma[j];
        }
    }
}

/* One token of the faithful recurrence for channel chan = h*P + p:
 *   out = D[h]*x; for n: h_n = decay*h_n + delta*B[g,n]*x; out += h_n*C[g,n]
 * with A_log per head (the reference) or per (head, state) (the Mamba-1
 * generalisation: decay indexed by n as well).
 * OXN/nsos/src/mamba2.cpp:2637-2666 */
static float scan_token(const float* x_row, const float* dt_row, const float* a_log,
                        int a_per_state, const float* B_row, const float* C_row,
                        const float* Dskip, int h, int p, int P, int N, int group,
                        float* state) {
    const int chan = h * P + p;
    const float xv = x_row[chan];
    float out = Dskip[h] * xv;
    float delta = 0.0f, decay = 0.0f;
    if (!a_per_state) orc_decay_terms(dt_row[h], a_log[h], &delta, &decay);
    for (int n = 0; n < N; ++n) {
        if (a_per_state) orc_decay_terms(dt_row[h], a_log[(int64_t)h * N + n], &delta, &decay);
        const float bx = (delta * B_row[group * N + n]) * xv;
        const float hv = fmaf(decay, state[(int64_t)chan * N + n], bx);
        state[(int64_t)chan * N + n] = hv;
        out = fmaf(hv, C_row[group * N + n], out);
    }
    return out;
}

/* Packed ragged forward scan.  Each sequence s covers tokens
 * [cu_seqlens[s], cu_seqlens[s+1]) and starts from initial_state[s] (or zeros);
 * final_state[s] receives the state after its last token (the reference reads
 * it as the last history row, mamba2.cpp:2814-2818).  Layouts: x, z, y
 * [T, H*P]; dt [T, H]; B, C [T, G*N]; A_log [H] or [H, N]; D [H];
 * states [num_seqs, H*P, N].  Gate: y = out * silu(z) (Tensor::silu_gate,
 * tensor.cpp:3323-3343).  OXN/nsos/src/mamba2.cpp:2602-2675 */
void orc_selective_scan(const float* x, const float* dt, const float* a_log,
                        int a_per_state, const float* B, const float* C,
                        const float* Dskip, const float* z, const int32_t* cu_seqlens,
                        int num_seqs, int H, int P, int N, int G,
                        const float* initial_state, float* y, float* final_state,
                        int gate_silu) {
    const int D = H * P;
    const int GS = G * N;
    const size_t one_state = (size_t)D * (size_t)N;
    float* state = (float*)malloc(sizeof(float) * one_state);
    for (int s = 0; s < num_seqs; ++s) {
        if (initial_state) memcpy(state, initial_state + (size_t)s * one_state, sizeof(float) * one_state);
        else memset(state, 0, sizeof(float) * one_state);
        for (int t = cu_seqlens[s]; t < cu_seqlens[s + 1]; ++t) {
            const float* xr = x + (int64_t)t * D;
            for (int h = 0; h < H; ++h) {
                const int group = (h * G) / H;
                for (int p = 0; p < P; ++p) {
                    float out = scan_token(xr, dt + (int64_t)t * H, a_log, a_per_state,
                                           B + (int64_t)t * GS, C + (int64_t)t * GS, Dskip,
                                           h, p, P, N, group, state);
                    const int chan = h * P + p;
                    if (gate_silu) out = out * orc_silu(z[(int64_t)t * D + chan]);
                    y[(int64_t)t * D + chan] = out;
                }
            }
        }
        if (final_state) memcpy(final_state + (size_t)s * one_state, state, sizeof(float) * one_state);
    }
    free(state);
}

/* Decode step over R independent rows: one token per row against its own
 * state [H*P, N], updated in place.  Same per-element math as the prefill.
 * OXN/nsos/src/mamba2.cpp:4097-4118 */
void orc_scan_step(const float* x, const float* dt, const float* a_log, int a_per_state,
                   const float* B, const float* C, const float* Dskip, const float* z,
                   int rows, int H, int P, int N, int G, float* state, float* y,
                   int gate_silu) {
    const int D = H * P;
    const int GS = G * N;
    for (int r = 0; r < rows; ++r) {
        float* st = state + (size_t)r * (size_t)D * (size_t)N;
        for (int h = 0; h < H; ++h) {
            const int group = (h * G) / H;
            for (int p = 0; p < P; ++p) {
                float out = scan_token(x + (int64_t)r * D, dt + (int64_t)r * H, a_log,
                                       a_per_state, B + (int64_t)r * GS, C + (int64_t)r * GS,
                                       Dskip, h, p, P, N, group, st);
                const int chan = h * P + p;
                if (gate_silu) out = out * orc_silu(z[(int64_t)r * D + chan]);
                y[(int64_t)r * D + chan] = out;
            }
        }
    }
}

/* ========================================================================
 * MoE routing / dispatch
 * ====================================================================== */

/* Tensor::softmax over the last axis: max-subtract, exp, in-order float sum,
 * multiply by 1/max(sum, 1e-8f).  OXN/nsos/src/tensor.cpp:3428-3450 */
void orc_softmax_rows(const float* logits, int rows, int cols, float* probs) {
    for (int r = 0; r < rows; ++r) {
        const float* src = logits + (int64_t)r * cols;
        float* dst = probs + (int64_t)r * cols;
        float mx = src[0];
        for (int j = 1; j < cols; ++j) mx = src[j] > mx ? src[j] : mx;
        float sum = 0.0f;
        for (int j = 0; j < cols; ++j) {
            dst[j] = expf(src[j] - mx);
            sum = sum + dst[j];
        }
        const float inv = 1.0f / (sum > 1e-8f ? sum : 1e-8f);
        for (int j = 0; j < cols; ++j) dst[j] = dst[j] * inv;
    }
}

/* Top-k by (value desc, index asc), renormalise by 1/max(sum of selected in
 * rank order, 1e-9f), zero the rest.  selected[r*k + rank] = expert id.
 * MoERouter::forward CPU path, OXN/nsos/src/jamba.cpp:8268-8297 */
void orc_topk_mask(float* weights, int rows, int experts, int k, int32_t* selected) {
    int32_t* rank = (int32_t*)malloc(sizeof(int32_t) * (size_t)experts);
    for (int r = 0; r < rows; ++r) {
        float* w = weights + (int64_t)r * experts;
        for (int e = 0; e < experts; ++e) rank[e] = e;
        /* selection sort of the first k ranks under the strict total order */
        for (int i = 0; i < k; ++i) {
            int best = i;
            for (int j = i + 1; j < experts; ++j) {
                const float a = w[rank[j]], b = w[rank[best]];
                if (a > b || (a == b && rank[j] < rank[best])) best = j;
            }
            const int32_t t = rank[i];
            rank[i] = rank[best];
            rank[best] = t;
        }
        /* the mask and renormalisation run only when k < experts (jamba.cpp:8268) */
        if (k < experts) {
            float sum = 0.0f;
            for (int i = 0; i < k; ++i) sum = sum + w[rank[i]];
            const float inv = 1.0f / (sum > 1e-9f ? sum : 1e-9f);
            for (int e = 0; e < experts; ++e) {
                int keep = 0;
                for (int i = 0; i < k; ++i) keep |= rank[i] == e;
                w[e] = keep ? w[e] * inv : 0.0f;
            }
        }
        if (selected)
            for (int i = 0; i < k; ++i) selected[(int64_t)r * k + i] = rank[i];
    }
    free(rank);
}

/* Padding rows of MoERouter::forward(x, valid_rows): after the top-k mask a row
 * whose valid byte is 0 gets all-zero weights (CPU path OXN/nsos/src/jamba.cpp:
 * 8299-8304; device path 8195-8214 through moe_zero_invalid_rows_kernel,
 * OXN/nsos/src/cuda/moe_kernels.cu:118-125, which reads 0 as padding) and no
 * selection (-1): the device dispatch takes only nonzero weights
 * (moe_count_per_expert_kernel / moe_ordered_assign_kernel,
 * OXN/nsos/src/cuda/moe_kernels.cu:226-235, 305-319). */
void orc_zero_invalid_rows(float* weights, int32_t* selected, const uint8_t* valid, int rows,
                           int experts, int k) {
    for (int r = 0; r < rows; ++r) {
        if (valid[r] != 0) continue;
        for (int e = 0; e < experts; ++e) weights[(int64_t)r * experts + e] = 0.0f;
        if (selected)
            for (int i = 0; i < k; ++i) selected[(int64_t)r * k + i] = -1;
    }
}

/* expert_loads of MoERouter::forward: loads[e] = sum over rows, in ascending order,
 * of the masked weights[r, e] (OXN/nsos/src/jamba.cpp:8299-8307, skipping padding
 * rows; the order of moe_load_ordered_kernel, OXN/nsos/src/cuda/moe_kernels.cu:
 * 108-116). */
void orc_expert_loads(const float* weights, const uint8_t* valid, int rows, int experts,
                      float* loads) {
    for (int e = 0; e < experts; ++e) loads[e] = 0.0f;
    for (int r = 0; r < rows; ++r) {
        if (valid && valid[r] == 0) continue;
        for (int e = 0; e < experts; ++e) loads[e] = loads[e] + weights[(int64_t)r * experts + e];
    }
}

/* Expert-major, rows-ascending dispatch of a selection [rows, k] (-1 = none):
 * each row joins the lists of its selected experts; offsets is the exclusive
 * scan of counts and perm[offsets[e] + i] is the i-th row routed to e.
 * JambaBlock::forward_moe, OXN/nsos/src/jamba.cpp:3882-3894 */
void orc_moe_dispatch_sel(const int32_t* sel, int rows, int experts, int k, int32_t* counts,
                          int32_t* offsets, int32_t* perm) {
    if (experts <= 0) return;
    for (int e = 0; e < experts; ++e) counts[e] = 0;
    for (int64_t i = 0; i < (int64_t)rows * k; ++i)
        if (sel[i] >= 0) counts[sel[i]]++;
    offsets[0] = 0;
    for (int e = 0; e < experts; ++e) offsets[e + 1] = offsets[e] + counts[e];
    int32_t* fill = (int32_t*)calloc((size_t)experts, sizeof(int32_t));
    for (int e = 0; e < experts; ++e)
        for (int r = 0; r < rows; ++r)
            for (int i = 0; i < k; ++i)
                if (sel[(int64_t)r * k + i] == e) perm[offsets[e] + fill[e]++] = r;
    free(fill);
}

/* The same dispatch from routing weights: each row's k highest-weighted experts
 * (orc_topk_mask's order).  OXN/nsos/src/jamba.cpp:3882-3894 */
void orc_moe_dispatch(const float* weights, int rows, int experts, int k,
                      int32_t* counts, int32_t* offsets, int32_t* perm) {
    float* tmp = (float*)malloc(sizeof(float) * (size_t)rows * (size_t)experts);
    int32_t* sel = (int32_t*)malloc(sizeof(int32_t) * (size_t)rows * (size_t)k);
    memcpy(tmp, weights, sizeof(float) * (size_t)rows * (size_t)experts);
    orc_topk_mask(tmp, rows, experts, k, sel);
    orc_moe_dispatch_sel(sel, rows, experts, k, counts, offsets, perm);
    free(sel);
    free(tmp);
}

/* Weighted combine in ascending expert order: out[r] starts at 0 and adds
 * expert_out[slot] * w[r,e] for e = 0..E-1 (0 for experts the row skipped).
 * OXN/nsos/src/jamba.cpp:3947-3969 */
void orc_moe_combine(const float* expert_out, const int32_t* perm, const int32_t* offsets,
                     const float* weights, int rows, int experts, int dim, float* out) {
    memset(out, 0, sizeof(float) * (size_t)rows * (size_t)dim);
    for (int e = 0; e < experts; ++e) {
        for (int s = offsets[e]; s < offsets[e + 1]; ++s) {
            const int r = perm[s];
            const float w = weights[(int64_t)r * experts + e];
            for (int d = 0; d < dim; ++d) {
                const float scaled = expert_out[(int64_t)s * dim + d] * w;
                out[(int64_t)r * dim + d] = out[(int64_t)r * dim + d] + scaled;
            }
        }
    }
}

/* ---- quantization-aware training ------------------------------------------
 * qat_fake_quant_ternary: inv = 1 / (scale + 1e-8f); v = w * inv;
 * out = (v > 0.5 ? 1 : v < -0.5 ? -1 : 0) * scale.
 * OXN/nsos/src/bitnet_gpu_dispatch.cpp:193-217 (CPU branch 209-216) */
void orc_qat_fake_quant_ternary(const float* w, int64_t n, float scale, float* out) {
    const float inv = 1.0f / (scale + 1e-8f);
    for (int64_t i = 0; i < n; ++i) {
        const float v = w[i] * inv;
        const float t = (v > 0.5f) ? 1.0f : ((v < -0.5f) ? -1.0f : 0.0f);
        out[i] = t * scale;
    }
}

/* qat_fake_quant_ternary_absmean: scale = tensor_abs_mean(w) + 1e-8f
 * (double sum, src/tensor.cpp:2095-2101), then the ternary fake-quant.
 * OXN/nsos/src/bitnet_gpu_dispatch.cpp:238-244 */
float orc_qat_fake_quant_ternary_absmean(const float* w, int64_t n, float* out) {
    const float scale = orc_absmean(w, n) + 1e-8f;
    orc_qat_fake_quant_ternary(w, n, scale, out);
    return scale;
}

/* qat_fake_quant_activations, per row: denom = max|x| + 1e-8f;
 * scale = q_max / denom; inv_scale = denom / q_max;
 * out = round(min(max(x * scale, -q_max), q_max)) * inv_scale (std::round).
 * OXN/nsos/src/bitnet_gpu_dispatch.cpp:262-281 */
void orc_qat_fake_quant_activations(const float* x, int M, int K, int bits, float* out) {
    const float q_max = bits <= 2 ? 1.0f : (float)((1 << (bits - 1)) - 1);
    for (int r = 0; r < M; ++r) {
        const float* row = x + (int64_t)r * K;
        float* orow = out + (int64_t)r * K;
        float mx = 0.0f;
        for (int j = 0; j < K; ++j) mx = fmaxf(mx, fabsf(row[j]));
        const float denom = mx + 1e-8f;
        const float scale = q_max / denom;
        const float inv_scale = denom / q_max;
        for (int j = 0; j < K; ++j) {
            float v = row[j] * scale;
            v = fminf(fmaxf(v, -q_max), q_max);
            orow[j] = roundf(v) * inv_scale;
        }
    }
}

/* qat_ste_clip_weight_grad: dW[i] = 0 where |w[i] * (1 / (scale + 1e-8f))| > 1.
 * OXN/nsos/src/bitnet_gpu_dispatch.cpp:300-307 */
void orc_qat_ste_clip(float* dW, const float* w, int64_t n, float scale) {
    const float inv = 1.0f / (scale + 1e-8f);
    for (int64_t i = 0; i < n; ++i)
        if (fabsf(w[i] * inv) > 1.0f) dW[i] = 0.0f;
}

/* ========================================================================
 * BitLinear float (quantization-sensitive) path and the packed STE backward
 * ====================================================================== */

/* Tensor::rmsnorm_backward (OXN/nsos/src/tensor.cpp:3997-4056) per row:
 *   sum_sq += x*x; dot += g*y  in index order: gcc -O3 -mavx -mfma forms the
 *   products of the first K - K%4 elements as rounded vector products (summed
 *   in order) and fuses the last K%4 into fma, as in Tensor::rmsnorm;
 *   dot /= K; inv_rms = 1/sqrt(sum_sq/K + eps); dx = (g - y*dot) * inv_rms with
 *   g - y*dot fused.  Pinned bit for bit against the reference build's output
 *   (tests/golden/tensor_ref.npz and oracle/_ref). */
void orc_rmsnorm_backward(const float* x, const float* g, const float* y, int rows, int cols,
                          float eps, float* dx) {
#pragma omp parallel for
    for (int r = 0; r < rows; ++r) {
        const int64_t base = (int64_t)r * cols;
        float sum_sq = 0.0f, dot = 0.0f;
        const int body = cols & ~3;
        for (int j = 0; j < body; ++j) {
            const float sq = x[base + j] * x[base + j];
            const float gy = g[base + j] * y[base + j];
            sum_sq = sum_sq + sq;
            dot = dot + gy;
        }
        for (int j = body; j < cols; ++j) {
            sum_sq = fmaf(x[base + j], x[base + j], sum_sq);
            dot = fmaf(g[base + j], y[base + j], dot);
        }
        const float k = (float)(cols > 1 ? cols : 1);
        dot = dot / k;
        const float inv_rms = 1.0f / sqrtf(sum_sq / k + eps);
        for (int j = 0; j < cols; ++j)
            dx[base + j] = fmaf(-y[base + j], dot, g[base + j]) * inv_rms;
    }
}

/* The float reference path BitLinear keeps for quantization-sensitive layers
 * (OXN/nsos/src/bitlinear.cpp:465-518): optional RMS_PERI input norm, then
 * x @ W^T, then *magnitude and +bias, each rounded.  The float matmul's
 * summation order belongs to the reference's matmul_nt; this restatement
 * accumulates in double (a tolerance oracle, checked against the reference
 * build's outputs in tests/golden/bitlinear_ref.npz). */
void orc_linear_f32(const float* x, int M, int K, int N, const float* w, int rms_input,
                    const float* magnitude, const float* bias, float* y) {
    float* xn = NULL;
    const float* src = x;
    if (rms_input) {
        xn = (float*)malloc(sizeof(float) * (size_t)M * (size_t)K);
        orc_rmsnorm(x, M, K, 1e-6f, xn);
        src = xn;
    }
#pragma omp parallel for
    for (int m = 0; m < M; ++m) {
        for (int n = 0; n < N; ++n) {
            double acc = 0.0;
            for (int k = 0; k < K; ++k)
                acc += (double)src[(int64_t)m * K + k] * (double)w[(int64_t)n * K + k];
            float v = (float)acc;
            if (magnitude) v = v * magnitude[n];
            if (bias) v = v + bias[n];
            y[(int64_t)m * N + n] = v;
        }
    }
    free(xn);
}

/* BitLinear::backward on the packed path: the straight-through estimator of
 * OXN/nsos/src/bitlinear.cpp:1191-1357, given what the forward saved.
 *   x         the layer input [M, K] (pre-norm)
 *   q, as     the int8 codes and act_scale the forward multiplied
 *   w         latent fp32 weights [N, K] (for the clip); codes their ternary
 *   grad      dL/dy [M, N]
 *   pre[i,j]  = float(acc) * (as[i] * ws)                (gemm without affine)
 *   dmag[j]   = sum_i grad[i,j] * pre[i,j]               (magnitude != NULL)
 *   dbias[j]  = sum_i grad[i,j]                          (dbias != NULL)
 *   gp        = grad * magnitude (or grad in exact-linear mode)
 *   dW[j,k]   = sum_i gp[i,j] * (q[i,k] * as[i]); 0 where |w / (ws + 1e-8f)| > 1
 *   d_act     = gp @ (codes * ws)
 *   dx        = rms_input ? rmsnorm_backward(x, d_act, rmsnorm(x)) : d_act
 * Sums accumulate in double: a tolerance oracle pinned by the reference build's
 * outputs (tests/golden/bitlinear_ref.npz). */
void orc_bitlinear_ste_backward(const float* x, const int8_t* q, const float* as,
                                const float* w, const int8_t* codes, float ws, int M, int K,
                                int N, int rms_input, const float* magnitude, const float* grad,
                                float* dx, float* dW, float* dmag, float* dbias) {
    float* gp = (float*)malloc(sizeof(float) * (size_t)M * (size_t)N);
    float* dact = (float*)malloc(sizeof(float) * (size_t)M * (size_t)K);
    for (int j = 0; j < N; ++j) {
        double sm = 0.0, sb = 0.0;
        for (int i = 0; i < M; ++i) {
            const float g = grad[(int64_t)i * N + j];
            if (magnitude) {
                int64_t acc = 0;
                for (int k = 0; k < K; ++k)
                    acc += (int64_t)q[(int64_t)i * K + k] * codes[(int64_t)j * K + k];
                const float pre = (float)acc * (as[i] * ws);
                sm += (double)(g * pre);
                gp[(int64_t)i * N + j] = g * magnitude[j];
            } else {
                gp[(int64_t)i * N + j] = g;
            }
            sb += (double)g;
        }
        if (dmag) dmag[j] = (float)sm;
        if (dbias) dbias[j] = (float)sb;
    }
    const float clip = ws + 1e-8f;
#pragma omp parallel for
    for (int j = 0; j < N; ++j) {
        for (int k = 0; k < K; ++k) {
            double acc = 0.0;
            for (int i = 0; i < M; ++i)
                acc += (double)gp[(int64_t)i * N + j] * (double)((float)q[(int64_t)i * K + k] * as[i]);
            const float wv = w[(int64_t)j * K + k];
            dW[(int64_t)j * K + k] = fabsf(wv / clip) > 1.0f ? 0.0f : (float)acc;
        }
    }
#pragma omp parallel for
    for (int i = 0; i < M; ++i) {
        for (int k = 0; k < K; ++k) {
            double acc = 0.0;
            for (int j = 0; j < N; ++j)
                acc += (double)gp[(int64_t)i * N + j] * (double)((float)codes[(int64_t)j * K + k] * ws);
            dact[(int64_t)i * K + k] = (float)acc;
        }
    }
    if (rms_input) {
        float* xn = (float*)malloc(sizeof(float) * (size_t)M * (size_t)K);
        orc_rmsnorm(x, M, K, 1e-6f, xn);
        orc_rmsnorm_backward(x, dact, xn, M, K, 1e-6f, dx);
        free(xn);
    } else {
        memcpy(dx, dact, sizeof(float) * (size_t)M * (size_t)K);
    }
    free(dact);
    free(gp);
}
