/*
 * nsosx.h -- C ABI of the MI355X (gfx950) hybrid-layer hot path.
 *
 * Plain pointers and sizes, no torch or C++ types.  Every device pointer is a
 * HIP device address; `stream` is a hipStream_t passed as void* (NULL = the
 * null stream).  Every call enqueues work on `stream` and returns without
 * synchronising; buffers are owned by the caller and must stay alive until
 * the enqueued work has finished.  Every entry point returns an nsosx_status;
 * on any status other than NSOSX_OK nothing was enqueued and no output was
 * touched.
 *
 * Citations are into OXN/nsos/ of vitorGgC569/reimagined and name the
 * reference interface each entry point replaces.
 *
 * Data formats shared with the reference:
 *   packed ternary weights  uint32 words, 16 codes per word, code j of a word
 *                           at bits 2j; -1 -> 0, 0 -> 1, +1 -> 2; flat over
 *                           the row-major [N, K] matrix; K % 16 == 0 so rows
 *                           are word-aligned.  Code 3 is reserved and decodes
 *                           to 0 (src/bitnet_adapter.cpp:31,570-606).
 *   activation codes        int8 [M, K] row-major, |code| <= 127.
 *   act_scale               float [M], (max|x| + 1e-8f) / q_max.
 */
#ifndef NSOSX_H
#define NSOSX_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum nsosx_status {
    NSOSX_OK = 0,
    NSOSX_ERR_INVALID = 1,   /* bad shape, null pointer or argument range */
    NSOSX_ERR_OVERFLOW = 2,  /* size product exceeds what the kernels index */
    NSOSX_ERR_RESERVED = 3,  /* packed weights hold the reserved code 3 */
    NSOSX_ERR_LAUNCH = 4,    /* the HIP runtime refused a launch or copy */
} nsosx_status;

typedef enum nsosx_dtype {
    NSOSX_F32 = 0,
    NSOSX_BF16 = 1,
} nsosx_dtype;

/* Last error text of the calling thread (never NULL). */
const char* nsosx_last_error(void);
/* Library version string. */
const char* nsosx_version(void);

/* ---------------------------------------------------------------------------
 * Host-side weight preparation (CPU, no device work).
 * ------------------------------------------------------------------------- */

/* BitLinear::pack_weights + quantize_weights (src/bitlinear.cpp:152-193,
 * 1359-1379): weight_scale = float(sum|w| / n in double) + 1e-8f; code = +1
 * if w/(weight_scale+1e-8f) > 0.5, -1 if < -0.5, else 0; packed as above.
 * w: float [N, K] host; packed: uint32 [N*K/16] host. */
int nsosx_pack_ternary(const float* w, int N, int K, uint32_t* packed, float* weight_scale);

/* Edge linear pack ("DGE1" v3 with the "EGI3" SHA-256 trailer, or legacy v2),
 * the reference's on-disk BitLinear format: JambaModel::load_edge_linear_pack
 * (src/jamba.cpp:1447-1620, field order 1345-1389, validation 556-616).  One
 * descriptor per layer; every vector is a byte offset into the caller's
 * buffer (zero-copy), the packed words in the format the GEMM/GEMV read. */
typedef struct nsosx_edge_layer {
    int32_t in_features;
    int32_t out_features;
    int32_t use_bias;
    int32_t sensitive;        /* 1: the layer also carries fp32 weights */
    float weight_scale;
    uint64_t packed_words;    /* ceil(in * out / 16) */
    uint64_t packed_offset;   /* uint32 [packed_words] */
    uint64_t magnitude_offset;/* f32 [out] */
    uint64_t bias_offset;     /* f32 [out] when use_bias */
    uint64_t alpha_offset;    /* f32 [in] (flat_alpha) */
    uint64_t beta_offset;     /* f32 [in] (flat_beta) */
    uint64_t sensitive_offset;/* f32 [out * in] when sensitive */
} nsosx_edge_layer;

/* Host parse + validation of a pack held in memory: magic, version, the v3
 * trailer (magic, payload length, SHA-256 of the payload), exact vector
 * lengths, finite values, positive finite weight_scale, no reserved code 3
 * (NSOSX_ERR_RESERVED), no trailing payload.  With more layers than
 * max_layers it returns NSOSX_ERR_OVERFLOW and the count in *num_layers (so
 * layers may be NULL with max_layers 0 to query it). */
int nsosx_edge_pack_parse(const uint8_t* data, uint64_t size, nsosx_edge_layer* layers,
                          int max_layers, int* num_layers, uint32_t* version);

/* SHA-256 (FIPS 180-4) of a host buffer as 64 lowercase hex digits plus NUL,
 * the digest the edge pack trailer carries (integrity::sha256_file_prefix,
 * src/sha256.cpp:221). */
int nsosx_sha256_hex(const uint8_t* data, uint64_t size, char* hex_out);

/* BitNetAdapter::unpack_weights_microsoft_style_to_i8
 * (src/bitnet_adapter.cpp:590-606): codes int8 [n] host. */
int nsosx_unpack_ternary(const uint32_t* packed, int64_t n, int8_t* codes);

/* Import check of BitLinear::import_packed_state (src/bitlinear.cpp:876-885),
 * on the device: *first_bad (device int64) receives the index of the first
 * reserved code, or -1.  Pre-upload weights go through this once. */
int nsosx_find_reserved_code(const uint32_t* packed, int64_t n_codes, int64_t* first_bad,
                             void* stream);

/* compute_weight_row_sums (src/bitlinear.cpp:36-73), on the device over the
 * packed words: sums[n] = sum_k w[n, k] (int32) with w decoded by the table
 * above.  packed: device [N * K / 16]; sums: device int32 [N]; K % 16 == 0. */
int nsosx_weight_row_sums(const uint32_t* packed, int N, int K, int32_t* sums, void* stream);

/* ---------------------------------------------------------------------------
 * BitLinear activations and ternary GEMM.
 * ------------------------------------------------------------------------- */

/* BitLinear::quantize_activations_bitnet on an AVX2 host
 * (src/bitlinear.cpp:240-291, src/bitlinear_quantize_avx2.cpp:65-103) plus the
 * GEMM's int8 clamp (src/bitnet_adapter_avx2.cpp:95-126); optionally preceded
 * by the RMS_PERI input norm (src/bitlinear.cpp:460-466 -> Tensor::rmsnorm,
 * src/tensor.cpp:3455-3492, eps 1e-6).  Replaces
 * launch_quantize_activations_bitnet_kernel (include/cuda/kernels.cuh).
 *   x: [M, K] f32 or bf16 (x_dtype), q: int8 [M, K], act_scale: f32 [M].
 *   bits in [2, 8]; rms_input 0/1.
 *   rms_workspace: f32 [M] device scratch, required when rms_input != 0. */
int nsosx_quantize_act_i8(const void* x, int x_dtype, int M, int K, int bits, int rms_input,
                          int8_t* q, float* act_scale, float* rms_workspace, void* stream);

/* Integer core + dequantizing epilogue of BitNetAdapter::gemm_158bit_i8
 * (src/bitnet_adapter.cpp:520-568, src/bitnet_adapter_avx2.cpp:52-158):
 *   acc[m,n] = sum_k q[m,k] * w[n,k]                       (exact int32)
 *   y[m,n]   = float(acc) * (act_scale[m] * weight_scale)
 *              then * magnitude[n], then + bias[n] (each rounded, no fma)
 * Replaces launch_bitnet_gemm / launch_bitnet_gemv_scaled /
 * launch_bitnet_apply_act_scales_kernel (include/cuda/kernels.cuh:106-110).
 * M = 1 runs the packed-weight streaming GEMV; 2 <= M <= 32 with K in
 * {1024, 2048, 4096} (ceil(M/16) * K <= 4096) the skinny MFMA kernel (one
 * decoded word feeds 16 tokens); other M <= 8 the GEMV; larger M the int8 MFMA
 * GEMM.
 *   y: [M, N] f32 or bf16 (y_dtype), may be NULL when acc_out is given.
 *   acc_out: int32 [M, N] or NULL (exposes the accumulators).
 *   magnitude, bias: f32 [N] or NULL. */
int nsosx_ternary_gemm(const int8_t* q, const float* act_scale, const uint32_t* packed,
                       float weight_scale, int M, int K, int N, const float* magnitude,
                       const float* bias, void* y, int y_dtype, int32_t* acc_out, void* stream);

/* Same contract, forcing one kernel: path 0 = streaming GEMV (M <= 8),
 * path 1 = MFMA GEMM (any M), path 2 = skinny MFMA (2 <= M <= 32, K in
 * {1024, 2048, 4096}, ceil(M/16) * K <= 4096, M * N < 2^29).  For tests and
 * measurement. */
int nsosx_ternary_gemm_path(const int8_t* q, const float* act_scale, const uint32_t* packed,
                            float weight_scale, int M, int K, int N, const float* magnitude,
                            const float* bias, void* y, int y_dtype, int32_t* acc_out,
                            int path, void* stream);

/* The packed weights of one [N, K] matrix rewritten into the layout the
 * prefill MFMA GEMM decodes fastest (an upload-time step, like the reference's
 * repack of its packed cache, src/bitlinear.cpp:628-643): within each 16-code
 * word, code k becomes its ternary value as a two's-complement 2-bit field
 * (-1 -> 3, 0 -> 0, +1 -> 1; the reserved code 3 -> 0) at bits
 * 8 (k % 4) + 6 - 2 (k / 4).  Words stay row-major, K / 16 per row.
 * packed, out: device uint32 [n_words] (distinct buffers). */
int nsosx_pack_mfma_layout(const uint32_t* packed, int64_t n_words, uint32_t* out,
                           void* stream);

/* nsosx_ternary_gemm's contract on weights in the MFMA layout above: the
 * int8 MFMA GEMM, or for decode batches the skinny path takes (2 <= M <= 32,
 * K in {1024, 2048, 4096}) the skinny MFMA kernel on the same words.
 * K % 128 == 0, K <= 264208 (the layout's operands are 64 x the ternary
 * values, so 64 * 127 * K must fit int32; larger K returns
 * NSOSX_ERR_OVERFLOW).  Same results bit for bit as nsosx_ternary_gemm on the
 * reference-layout words. */
int nsosx_ternary_gemm_mfma(const int8_t* q, const float* act_scale, const uint32_t* packed_mfma,
                            float weight_scale, int M, int K, int N, const float* magnitude,
                            const float* bias, void* y, int y_dtype, int32_t* acc_out,
                            void* stream);

/* bitnet_gemm_158bit_gpu (include/bitnet_gpu_dispatch.h:46-51,
 * src/bitnet_gpu_dispatch.cpp:65-174): quantize x then ternary GEMM.
 * q_workspace: int8 [M, K]; scale_workspace: f32 [M];
 * rms_workspace: f32 [M] (only with rms_input). */
int nsosx_bitlinear_forward(const void* x, int x_dtype, const uint32_t* packed,
                            float weight_scale, int M, int K, int N, int precision_bits,
                            int rms_input, const float* magnitude, const float* bias, void* y,
                            int y_dtype, int8_t* q_workspace, float* scale_workspace,
                            float* rms_workspace, void* stream);

/* No counterpart in the reference.  nsosx_bitlinear_forward for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops
 * that forbid hipMalloc): the int8 codes, act_scale and RMS workspace live in
 * a library-owned static device array of nsosx_bitlinear_forward_noalloc_max_bytes()
 * bytes (8 MiB) per GPU, held until the process ends; no allocation happens.
 * The workspace takes round256(M*K) + 2*round256(4*M) bytes; larger shapes
 * return NSOSX_ERR_OVERFLOW.  Every call on one GPU shares that array, so
 * calls that overlap on one GPU (different streams, or different host threads)
 * race; calls enqueued on one stream are ordered and safe.  The first call on
 * each device looks up the array's device address and must be made outside
 * HIP graph capture (under capture it returns NSOSX_ERR_INVALID); later calls
 * may be captured and replayed. */
int64_t nsosx_bitlinear_forward_noalloc_max_bytes(void);
int nsosx_bitlinear_forward_noalloc(const void* x, int x_dtype, const uint32_t* packed,
                                    float weight_scale, int M, int K, int N, int precision_bits,
                                    int rms_input, const float* magnitude, const float* bias,
                                    void* y, int y_dtype, void* stream);

/* The float reference path BitLinear keeps for quantization-sensitive layers
 * (src/bitlinear.cpp:465-518): the faithful Mamba-2 block's B / C / dt
 * projections (src/mamba2.cpp:588-599, 655-662, exact-linear mode: no input
 * norm, no magnitude; dt with its bias) and the MoE router's gate
 * (src/jamba.cpp:8086-8098: RMS_PERI and magnitude).
 *   y = (rms_input ? rmsnorm(x, 1e-6) : x) @ w^T, then * magnitude[n], then + bias[n]
 * x: [M, K] (x_dtype); w: f32 [N, K]; y: [M, N] (y_dtype); magnitude, bias:
 * f32 [N] or NULL; rms_workspace: f32 [M] when rms_input (required; the
 * skinny shapes below do not use it).  K % 4 == 0.
 * The dot products accumulate in fp32 in an order of their own: N <= 64 with
 * M > 16 on v_mfma_f32_16x16x4_f32 in one pass over x, the RMS sums of
 * squares taken on the way and 1 / rms applied to the dot products (equal to
 * the dot of the normalised row to rounding); other shapes with the
 * normalised input x * inv formed bit for bit as Tensor::rmsnorm, on
 * v_mfma_f32_32x32x2_f32 or, for N <= 16 or M <= 16, a wave reduction. */
int nsosx_linear_f32(const void* x, int x_dtype, int M, int K, const float* w, int N,
                     int rms_input, const float* magnitude, const float* bias, void* y,
                     int y_dtype, float* rms_workspace, void* stream);

/* BitLinear::backward on the packed path: the straight-through estimator of
 * src/bitlinear.cpp:1191-1357, given what the forward saved:
 *   x          the layer input [M, K] (x_dtype; read only when rms_input)
 *   q, act_scale  the int8 codes [M, K] and scales [M] the forward multiplied
 *   w_latent   f32 [N, K] latent weights (for the clip); packed their ternary
 *   grad       f32 [M, N], dL/dy
 *   pre        = acc * (act_scale * weight_scale)           (GEMM without affine)
 *   dmag[n]    = sum_m grad * pre          (magnitude given; dmag may be NULL)
 *   dbias[n]   = sum_m grad                (NULL: no bias)
 *   gp         = grad * magnitude (grad in exact-linear mode, magnitude NULL)
 *   dW[n, k]   = sum_m gp[m, n] * (q[m, k] * act_scale[m]), 0 where
 *                |w_latent / (weight_scale + 1e-8f)| > 1
 *   d_act      = gp @ (ternary * weight_scale)
 *   dx         = rms_input ? rmsnorm_backward(x, d_act, rmsnorm(x)) : d_act
 * All outputs f32.  K % 16 == 0, N % 4 == 0.  workspace: device,
 * nsosx_bitlinear_ste_backward_workspace(M, K, N, rms_input) bytes, 256-byte
 * aligned.  Sums run in fp32 in an order of their own (tolerance parity). */
int64_t nsosx_bitlinear_ste_backward_workspace(int M, int K, int N, int rms_input);
int nsosx_bitlinear_ste_backward(const void* x, int x_dtype, const int8_t* q,
                                 const float* act_scale, const float* w_latent,
                                 const uint32_t* packed, float weight_scale, int M, int K, int N,
                                 int rms_input, const float* magnitude, const float* grad,
                                 float* dx, float* dW, float* dmag, float* dbias,
                                 void* workspace, void* stream);

/* One borrowed descriptor per weight set, the C shape of nsos::GpuLinearView
 * (include/gpu_linear_view.h:8-26) restricted to the packed path. */
typedef struct nsosx_linear_view {
    const uint32_t* packed;   /* device, [outputs * inputs / 16] */
    const float* magnitude;   /* device [outputs] or NULL */
    const float* bias;        /* device [outputs] or NULL */
    int inputs;
    int outputs;
    float weight_scale;
} nsosx_linear_view;

/* Grouped decode GEMV: `groups` independent ternary GEMVs in one launch, the
 * role of launch_grouped_decode_projections (include/cuda/kernels.cuh:27-29).
 * Group g multiplies q + g*q_stride (int8 [M, inputs]) with views[g] and
 * writes y + g*y_stride elements ([M, outputs], y_dtype); act_scale + g *
 * scale_stride holds the group's M scales (zero strides share one input
 * across the groups, as the decode projections of one token do).  M <= 8.
 * views_dev: device array of `groups` descriptors (the caller uploads it once
 * and reuses it). */
int nsosx_grouped_gemv(const nsosx_linear_view* views_dev, int groups, const int8_t* q,
                       int64_t q_stride, const float* act_scale, int64_t scale_stride, int M,
                       void* y, int64_t y_stride, int y_dtype, void* stream);

/* A decode projection (GpuLinearView, include/gpu_linear_view.h:8-25): a packed
 * ternary BitLinear (packed != NULL, activation_bits 2..8) or a float linear
 * (weight f32 [outputs, inputs], activation_bits 0), optional magnitude and bias,
 * optional RMS_PERI input norm. */
typedef struct nsosx_decode_view {
    const float* weight;      /* device f32 [outputs, inputs] or NULL */
    const uint32_t* packed;   /* device [outputs * inputs / 16] or NULL */
    const float* magnitude;   /* device [outputs] or NULL */
    const float* bias;        /* device [outputs] or NULL */
    int inputs;
    int outputs;
    int activation_bits;      /* 0: unquantized activations (float views) */
    int rms_input;
    float weight_scale;
} nsosx_decode_view;

/* GpuProjectionGroup::forward / launch_grouped_decode_projections
 * (src/gpu_projection_group.cpp:12-49, src/cuda/moe_kernels.cu:779-784): one
 * input row (in_dtype, each view reads its first `inputs` elements) through
 * `groups` projections in one launch; view g writes output + g * output_stride
 * ([outputs_g], out_dtype).  With the CPU path's numerics, as every other
 * entry: a packed view quantizes the row like nsosx_quantize_act_i8 (RMS_PERI
 * when rms_input) and runs the ternary GEMV, so its output equals
 * nsosx_bitlinear_forward at M = 1 bit for bit; a float view equals
 * nsosx_linear_f32 at M = 1 bit for bit.  Each workgroup of a packed view
 * quantizes the row itself (no prepared buffer).  A packed view needs
 * inputs % 64 == 0 and inputs <= 4096; a float view inputs % 4 == 0 and
 * 16-byte aligned rows; a view that does not meet them is skipped.
 * views_dev: device array of `groups` descriptors. */
int nsosx_grouped_decode_projections(const nsosx_decode_view* views_dev, int groups,
                                     const void* input, int in_dtype, void* output,
                                     int64_t output_stride, int out_dtype, void* stream);

/* ---------------------------------------------------------------------------
 * Mamba selective scan.
 * ------------------------------------------------------------------------- */

/* Depthwise causal convolution restarted at every cu_seqlens boundary, plus
 * bias and SiLU (src/mamba2.cpp:1056-1076, 2437-2446):
 *   out[t,c] = silu(bias[c] + sum_{j<W} w[c,j] * in[t-(W-1)+j, c])
 * in: [T, channels] with row stride in_stride elements (in_dtype);
 * out: [T, channels] contiguous (out_dtype).  w: f32 [channels, W]. */
int nsosx_conv1d_causal(const void* in, int in_dtype, int64_t in_stride, const float* weight,
                        const float* bias, const int32_t* cu_seqlens, int num_seqs,
                        int total_tokens, int channels, int width, int apply_silu, void* out,
                        int out_dtype, void* stream);

/* Packed ragged selective-scan forward: the faithful recurrence of
 * src/mamba2.cpp:2602-2675 (GPU twin src/cuda/mamba_kernels.cu:1690-1754)
 * with the decay of mamba_decay_terms (src/mamba2.cpp:443-473), generalised
 * to A_log per (head, state) when a_per_state != 0 (Mamba-1 A[D, N]).
 * For each sequence s (tokens cu_seqlens[s] .. cu_seqlens[s+1]-1), head h,
 * channel c = h*P + p, state n, group g = h*G/H:
 *   delta = softplus(dt[t,h]);  decay = exp(-delta * exp(A_log[h(,n)]))
 *   state = decay * state + (delta * B[t,g,n]) * x[t,c]
 *   y[t,c] = D[h] * x[t,c] + sum_n state * C[t,g,n]
 *   y[t,c] *= silu(z[t,c])                              (when z != NULL)
 * Layouts (row-major, act_dtype for x, dt, B, C, z, y; f32 for the rest):
 *   x, z, y [T, H*P] with row strides x_stride, z_stride (y contiguous);
 *   dt [T, H]; B, C [T, G*N]; A_log [H] or [H, N]; D [H];
 *   initial_state, final_state f32 [num_seqs, H*P, N] or NULL.
 * N <= 64. */
int nsosx_selective_scan_fwd(const void* x, int64_t x_stride, const void* dt, const float* A_log,
                             int a_per_state, const void* B, const void* C, const float* D,
                             const void* z, int64_t z_stride, const int32_t* cu_seqlens,
                             int num_seqs, int total_tokens, int H, int P, int N, int G,
                             int act_dtype, const float* initial_state, float* final_state,
                             void* y, void* stream);

/* The scan with the depthwise causal convolution + bias + SiLU of the
 * Mamba block fused into its input staging (src/mamba2.cpp:1056-1076,
 * 2437-2446 feeding 2602-2675): x_raw is the convolution's input (row stride
 * x_stride), conv_w f32 [H*P, conv_width] (conv_width <= 8), conv_b f32
 * [H*P] or NULL; the convolution restarts at every sequence start.  The D
 * skip uses the convolved x.  Other arguments as nsosx_selective_scan_fwd;
 * channels per group must be a multiple of 64. */
int nsosx_conv_scan_fwd(const void* x_raw, int64_t x_stride, const float* conv_w,
                        const float* conv_b, int conv_width, const void* dt, const float* A_log,
                        int a_per_state, const void* B, const void* C, const float* D,
                        const void* z, int64_t z_stride, const int32_t* cu_seqlens, int num_seqs,
                        int total_tokens, int H, int P, int N, int G, int act_dtype,
                        const float* initial_state, float* final_state, void* y, void* stream);

/* The scan (x_raw through the causal conv when conv_w != NULL, as
 * nsosx_conv_scan_fwd; else as nsosx_selective_scan_fwd) with a launch plan
 * built on the device:
 *   - 65 to 512 sequences: one pre-pass ranks them longest-first for dispatch
 *     (up to 64 each workgroup ranks them itself; above 512 they run in
 *     dispatch order, no ranking at all);
 *   - chunk_tokens > 0 (>= 4): the time-chunked scan.  Every sequence splits
 *     into chunks of chunk_tokens tokens; a first pass runs each chunk's
 *     recurrence from zero and records its end state and summed delta, a
 *     combine carries the states across chunk boundaries (the decay product of
 *     a chunk is exp of its summed exponents), and a second pass runs each
 *     chunk from its carried state, its causal conv window taken from the
 *     sequence's previous tokens.  For batches whose sequences x 16-channel
 *     blocks cannot fill the GPU (one long prefill).  Needs channels per group
 *     a multiple of 64 and conv width <= 8 (any N <= 64, the faithful block's
 *     d_state 64 included), or, with N <= 16, a multiple of 16 and conv width
 *     <= 4.  Outputs equal the sequential scan to rounding (the carried states
 *     differ by a few ulp);
 *   - chunk_tokens == 0: never chunk; -1: chunk when sequences x (H*P/16) <
 *     2048 and the sequences are at least two chunks long (chunk size aiming
 *     at 8192 waves, at least 64 tokens).
 * workspace: device, nsosx_scan_fwd_workspace(num_seqs, total_tokens, H, P,
 * N, chunk_tokens) bytes, 256-byte aligned.  Other arguments as above. */
int64_t nsosx_scan_fwd_workspace(int num_seqs, int total_tokens, int H, int P, int N,
                                 int chunk_tokens);
int nsosx_scan_fwd_planned(const void* x, int64_t x_stride, const float* conv_w,
                           const float* conv_b, int conv_width, const void* dt,
                           const float* A_log, int a_per_state, const void* B, const void* C,
                           const float* D, const void* z, int64_t z_stride,
                           const int32_t* cu_seqlens, int num_seqs, int total_tokens, int H,
                           int P, int N, int G, int act_dtype, const float* initial_state,
                           float* final_state, void* y, int chunk_tokens, void* workspace,
                           void* stream);

/* Decode step over `rows` independent sequences, one token each, state
 * updated in place (src/mamba2.cpp:4038-4125; GPU twin
 * launch_mamba2_faithful_step, src/cuda/mamba_kernels.cu:3332-3419).
 * x, z, y [rows, H*P]; dt [rows, H]; B, C [rows, G*N] (act_dtype);
 * state f32 [rows, H*P, N]. */
int nsosx_selective_scan_step(const void* x, const void* dt, const float* A_log, int a_per_state,
                              const void* B, const void* C, const float* D, const void* z,
                              int rows, int H, int P, int N, int G, int act_dtype, float* state,
                              void* y, void* stream);

/* The faithful Mamba-2 decode step after its projections, in one launch
 * (Mamba2SSD streaming step, src/mamba2.cpp:4038-4125 from the conv ring to
 * out_proj's input; GPU twins launch_mamba2_faithful_conv_step and
 * launch_mamba2_faithful_step, src/cuda/mamba_kernels.cu:3332-3419, then the
 * gated norm and BitLinear::quantize_activations_bitnet, src/bitlinear.cpp:240-291
 * with src/bitlinear_quantize_avx2.cpp:65-103): per row,
 *   conv ring step + SiLU over the inner + 2*G*N channels x | B | C;
 *   state = decay * state + delta * B * x; y = D * x + state . C;
 *   normed = RMSNorm(y * SiLU(z), eps) * norm_w;
 *   act_scale = (absmax(normed) + 1e-8) / q_max, q = round(normed / act_scale)
 *   (q_max = 2^(act_bits-1) - 1, 1 at 2 bits), the input of a ternary GEMV.
 * Two launches: the conv / state step over 64-channel slices of each row, then
 * the B / C ring shift, norm and quantization per row.
 * x, z [rows, H*P] and y [rows, H*P] (written: the pre-gate output, the norm's
 * input) in act_dtype; B, C [rows, G*N] and dt [rows, H] (dt bias included) in act_dtype,
 * sharing the row stride bcdt_stride; conv_w f32 [H*P + 2*G*N, conv_width],
 * conv_b f32 [H*P + 2*G*N] or NULL; ring f32 [rows, conv_width - 1, H*P + 2*G*N]
 * (the reference's single ring); A_log, D f32 [H]; norm_w f32 [H*P] or NULL;
 * state f32 [rows, H*P, N], 16-byte aligned; q int8 [rows, H*P];
 * act_scale f32 [rows].  Limits: rows <= 65535, H*P <= 8192, G*N <= 1024,
 * N in {4, 8, 16, 32, 64} (the reference's MAX_N is 64), 1 <= conv_width <= 4.  The values equal nsosx_conv_step (x, B, C) +
 * nsosx_selective_scan_step + nsosx_rmsnorm_gated + nsosx_quantize_act_i8 bit
 * for bit when H*P is a multiple of 512 up to 4096 (the gated norm's register
 * path sums in the same order); otherwise to that sum's rounding. */
int nsosx_mamba2_step(const void* x, const void* z, const void* B, const void* C, const void* dt,
                      int64_t bcdt_stride, const float* conv_w, const float* conv_b,
                      int conv_width, float* ring, const float* A_log, const float* D,
                      const float* norm_w, float eps, int rows, int H, int P, int N, int G,
                      int act_dtype, float* state, void* y, int8_t* q, float* act_scale,
                      int act_bits, void* stream);

/* nsosx_mamba2_step and then the block's out_proj (Mamba2SSD's ternary out_proj in
 * exact-linear mode, src/mamba2.cpp:514 and 4121; bitnet_gemm_158bit_gpu semantics)
 * on its codes: out [rows, out_features] (out_dtype) = the ternary GEMM of q with
 * out_packed [out_features, H*P / 16] words and out_weight_scale, times
 * out_magnitude and plus out_bias where given.  One row with H*P % 64 == 0 and
 * H*P <= 4096 takes two launches (the out_proj GEMV forms the norm and codes itself
 * as its prologue); otherwise nsosx_mamba2_step + nsosx_ternary_gemm.  Either way y,
 * q and act_scale are written as by nsosx_mamba2_step, with the same values. */
int nsosx_mamba2_step_out(const void* x, const void* z, const void* B, const void* C,
                          const void* dt, int64_t bcdt_stride, const float* conv_w,
                          const float* conv_b, int conv_width, float* ring, const float* A_log,
                          const float* D, const float* norm_w, float eps, int rows, int H, int P,
                          int N, int G, int act_dtype, float* state, void* y, int8_t* q,
                          float* act_scale, int act_bits, const uint32_t* out_packed,
                          float out_weight_scale, int out_features, const float* out_magnitude,
                          const float* out_bias, void* out, int out_dtype, void* stream);

/* ---------------------------------------------------------------------------
 * Top-k MoE routing.
 * ------------------------------------------------------------------------- */

/* MoERouter::forward(x, valid_rows) from logits (src/jamba.cpp:8140-8319):
 * softmax (src/tensor.cpp:3428-3450), top-k by (probability desc, index asc),
 * renormalised by 1/max(sum, 1e-9f); padding rows zeroed; then the
 * expert-major, rows-ascending dispatch of JambaBlock::forward_moe
 * (src/jamba.cpp:3882-3894; the device path's ordered assignment,
 * src/cuda/moe_kernels.cu:305-319).
 *   logits f32 [rows, E]; weights f32 [rows, E] (masked, renormalised);
 *   valid_rows uint8 [rows], device, or NULL (every row valid): a row whose
 *   byte is 0 is padding, as launch_moe_zero_invalid_rows_kernel reads the
 *   mask (src/cuda/moe_kernels.cu:118-125).  A padding row gets all-zero
 *   weights, selected -1 and slot_of -1, takes no slot in counts / offsets /
 *   perm, and nsosx_moe_combine writes it as zeros.  MoERouter::forward
 *   rejects a host mask holding any value other than 0 or 1 before it is
 *   uploaded (src/jamba.cpp:8145-8153); the C++ and Python mirrors of this
 *   entry do the same.
 *   selected int32 [rows, k] (rank order); counts int32 [E];
 *   offsets int32 [E+1] (exclusive scan; offsets[E] = valid rows * k);
 *   perm int32 [rows*k] (slot -> row; the first offsets[E] entries are set);
 *   slot_of int32 [rows, k]: slot_of[r, i] is the slot of selected[r, i]
 *   (rank order), so perm[slot_of[r, i]] == r.
 *   loads f32 [E] or NULL: expert_loads, loads[e] = sum over rows in
 *   ascending order of weights[r, e] (src/jamba.cpp:8299-8307, the order of
 *   launch_moe_load_ordered_kernel, src/cuda/moe_kernels.cu:108-116).
 *   workspace: int32, nsosx_moe_route_workspace(rows, E) elements.
 * counts, offsets, perm, slot_of and workspace all NULL: selection only
 * (weights and selected, one launch), what the sparse decode consumes.
 * E <= 64, any 0 < k <= E (rows * k < 2^31). */
int64_t nsosx_moe_route_workspace(int rows, int experts);
int nsosx_moe_route(const float* logits, const uint8_t* valid_rows, int rows, int experts, int k,
                    float* weights, int32_t* selected, int32_t* counts, int32_t* offsets,
                    int32_t* perm, int32_t* slot_of, float* loads, int32_t* workspace,
                    void* stream);

/* Grouped ternary GEMM over expert segments: for each expert e the rows
 * perm[offsets[e] .. offsets[e+1]) of q (int8 [rows_in, K], gathered through
 * perm when gather != 0, else read as the slot-ordered q itself) multiply
 * views[e]; the result goes to slot order y [slots, N] with the view's
 * epilogue and then, when squared_relu != 0, max(v,0)^2 (Tensor::squared_relu,
 * src/tensor.cpp:3209-3226).  act_scale is indexed like q.
 * offsets is a device array.  max_rows_per_expert bounds any expert's rows;
 * total_rows (offsets[experts], or an upper bound; 0 = unknown) lets the launch
 * cover only the experts' real row tiles, found on the device from the offsets
 * (without it every expert is given max_rows_per_expert rows of workgroups). */
int nsosx_grouped_ternary_gemm(const nsosx_linear_view* views_dev, int experts,
                               const int32_t* offsets, const int32_t* perm, int gather,
                               const int8_t* q, const float* act_scale, int K, int N,
                               int max_rows_per_expert, int total_rows, int squared_relu,
                               void* y, int y_dtype, void* stream);

/* nsosx_grouped_ternary_gemm on views whose packed words are in the MFMA
 * layout (nsosx_pack_mfma_layout), launching only the experts' real row tiles.
 * total_rows sizes the launch and is required: offsets[experts] or an upper
 * bound, > 0 (0, which nsosx_grouped_ternary_gemm reads as "unknown", is
 * NSOSX_ERR_INVALID here: with no row bound the grid cannot be sized; a routing
 * with no rows needs no call).  K % 128 == 0, K <= 264208 (as
 * nsosx_ternary_gemm_mfma), <= 1024 experts.  Same results bit for bit. */
int nsosx_grouped_ternary_gemm_mfma(const nsosx_linear_view* views_dev, int experts,
                                    const int32_t* offsets, const int32_t* perm, int gather,
                                    const int8_t* q, const float* act_scale, int K, int N,
                                    int total_rows, int squared_relu, void* y, int y_dtype,
                                    void* stream);

/* nsosx_grouped_ternary_gemm_mfma with a workspace for a split-K tail: when the
 * launch's last round of tiles would leave at least three quarters of the
 * resident workgroups idle and K >= 2048 (the routed config-5 down GEMM: 528
 * tiles on 512), those tiles are split along K over 2-8 workgroups each, their
 * int32 partial sums go to the workspace and a second launch adds them and
 * applies the epilogue.
 * Integer partial sums: the same bits as nsosx_grouped_ternary_gemm_mfma.  The
 * same arguments and checks, plus workspace (device, 16-byte aligned) of at
 * least nsosx_grouped_ternary_gemm_mfma_workspace() bytes (2 x CUs x 128 KiB on
 * the current device; -1 without a device).  Two launches on `stream`; calls
 * sharing a workspace must not overlap.  This entry has no counterpart in the
 * reference (whose per-expert loop has no tail to balance). */
int64_t nsosx_grouped_ternary_gemm_mfma_workspace(void);
int nsosx_grouped_ternary_gemm_mfma_ws(const nsosx_linear_view* views_dev, int experts,
                                       const int32_t* offsets, const int32_t* perm, int gather,
                                       const int8_t* q, const float* act_scale, int K, int N,
                                       int total_rows, int squared_relu, void* y, int y_dtype,
                                       void* workspace, int64_t workspace_bytes, void* stream);

/* Weighted combine in ascending expert order (src/jamba.cpp:3947-3969):
 * out[r] = sum over the row's selected experts, lowest id first, of
 * expert_out[slot] * weights[r, e], starting from 0.
 * expert_out [slots, dim] (in_dtype), out [rows, dim] (out_dtype).
 * A row with selected[r, 0] < 0 (a padding row of nsosx_moe_route) is written
 * as zeros.  slot_of NULL: the slot of (row r, choice i) is r * k + i.  rows <= 65535 unless
 * dim % 4 == 0 and expert_out / out are 16-byte aligned (8 with both bf16). */
int nsosx_moe_combine(const void* expert_out, int in_dtype, const int32_t* slot_of,
                      const int32_t* selected, const float* weights, int rows, int experts, int k,
                      int dim, void* out, int out_dtype, void* stream);

/* Sparse MoE decode, the role of launch_moe_sparse_decode
 * (src/cuda/moe_kernels.cu:786-795) with forward_moe's semantics
 * (src/jamba.cpp:3865-3972): for each row and each of its k routed experts
 * (selected [rows, k], weights [rows, experts] from nsosx_moe_route), the
 * expert's up BitLinear -> squared ReLU -> down BitLinear as grouped GEMVs
 * over (row, expert) pairs, then the ascending-expert weighted combine.  x:
 * [rows, dim] (x_dtype); out [rows, dim] (out_dtype); rows * k <= 65535.
 * workspace: device, nsosx_moe_sparse_decode_workspace(rows, k, dim, hidden)
 * bytes. */
int64_t nsosx_moe_sparse_decode_workspace(int rows, int k, int dim, int hidden);
int nsosx_moe_sparse_decode(const nsosx_linear_view* up_views,
                            const nsosx_linear_view* down_views, int experts, int k,
                            const int32_t* selected, const float* weights, const void* x,
                            int x_dtype, int rows, int dim, int hidden, int rms_input,
                            void* workspace, void* out, int out_dtype, void* stream);

/* ---------------------------------------------------------------------------
 * Row norms of the hybrid block and the decode conv ring.
 * ------------------------------------------------------------------------- */

/* Gated RMSNorm epilogue RMSNorm(y * SiLU(z)) * gamma (src/mamba2.cpp:2677-2680,
 * launch_mamba_gated_rmsnorm src/cuda/mamba_kernels.cu:3421-3445); with z NULL
 * it is Tensor::rmsnorm (src/tensor.cpp:3455-3492) times gamma; gamma NULL is
 * a unit weight.  y, z: [rows, dim] (act_dtype); out: [rows, dim] (out_dtype).
 * The sum of squares is reduced in fp32 across the row in tree order. */
int nsosx_rmsnorm_gated(const void* y, const void* z, const float* gamma, int rows, int dim,
                        float eps, int act_dtype, void* out, int out_dtype, void* stream);

/* nsosx_rmsnorm_gated followed by the out_proj BitLinear's int8 input quantization
 * (quantize_activations_bitnet without RMS_PERI, src/bitlinear.cpp:240-291), as in
 * Mamba2SSD::forward_faithful (src/mamba2.cpp:2677-2681): the codes quantize the
 * normed values as stored in out_dtype.  q int8 [rows, dim], act_scale f32 [rows].
 * For dim % 512 == 0, dim <= 4096 and 16-byte aligned buffers one pass, and out
 * may be NULL (the normed rows are then not stored); otherwise the two passes of
 * nsosx_rmsnorm_gated + nsosx_quantize_act_i8 and out is required. */
int nsosx_rmsnorm_gated_quant(const void* y, const void* z, const float* gamma, int rows, int dim,
                              float eps, int act_dtype, void* out, int out_dtype, int bits,
                              int8_t* q, float* act_scale, void* stream);

/* Residual add and the next block norm of JambaBlock::forward
 * (src/jamba.cpp:3253, 3286-3290, 3316): residual_out = x + delta (act_dtype);
 * when norm_out is not NULL, norm_out = rmsnorm(residual_out, eps) * gamma
 * (gamma NULL = unit).  All buffers [rows, dim]. */
int nsosx_add_rmsnorm(const void* x, const void* delta, const float* gamma, int rows, int dim,
                      float eps, int act_dtype, void* residual_out, void* norm_out, void* stream);

/* Decode conv ring step, the role of launch_mamba2_faithful_conv_step
 * (src/cuda/mamba_kernels.cu:3332-3374; CPU src/mamba2.cpp:4072-4090):
 *   v = bias[c] + sum_{j<W} w[c,j] * (j < W-1 ? ring[r][j][c] : x[r,c])
 *   out[r,c] = apply_silu ? silu(v) : v; ring[r] shifts one slot and takes x[r,c].
 * x: [rows, channels] with row stride x_stride; ring: f32 [rows, W-1, channels]
 * (unused when W == 1); weight f32 [channels, W]; bias f32 [channels] or NULL. */
int nsosx_conv_step(const void* x, int x_dtype, int64_t x_stride, int rows, int channels,
                    const float* weight, const float* bias, int width, float* ring,
                    int apply_silu, void* out, int out_dtype, void* stream);

/* ---------------------------------------------------------------------------
 * Quantization-aware training: fake-quant forward and the STE weight-gradient
 * clip, bit-exact with the CPU path.  All tensors f32 on the device.
 * ------------------------------------------------------------------------- */

/* qat_fake_quant_ternary (src/bitnet_gpu_dispatch.cpp:193-217;
 * launch_fake_quant_ternary_kernel include/cuda/kernels.cuh:506):
 *   v = w * (1 / (scale + 1e-8f)); out = (v > 0.5 ? 1 : v < -0.5 ? -1 : 0) * scale.
 * scale finite and > 0. */
int nsosx_qat_fake_quant_ternary(const float* w, int64_t n, float scale, float* out,
                                 void* stream);

/* qat_fake_quant_ternary_absmean (src/bitnet_gpu_dispatch.cpp:219-245;
 * launch_fake_quant_ternary_absmean_kernel kernels.cuh:510): scale =
 * float(sum |w| / n, summed in double) + 1e-8f written to scale_out (device,
 * one float), then the fake-quant above with that scale; no host sync.
 * workspace: device, nsosx_qat_absmean_workspace(n) bytes. */
int64_t nsosx_qat_absmean_workspace(int64_t n);
int nsosx_qat_fake_quant_ternary_absmean(const float* w, int64_t n, float* out,
                                         float* scale_out, void* workspace, void* stream);

/* qat_fake_quant_activations (src/bitnet_gpu_dispatch.cpp:247-282;
 * launch_fake_quant_activations_kernel kernels.cuh:518), per row of x [M, K]:
 * denom = max|x| + 1e-8f; v = clamp(x * (q_max / denom), -q_max, q_max);
 * out = round_half_away(v) * (denom / q_max); q_max = 2^(bits-1) - 1 (1 for
 * bits = 2); precision_bits in [2, 8]. */
int nsosx_qat_fake_quant_activations(const float* x, int M, int K, int precision_bits,
                                     float* out, void* stream);

/* qat_ste_clip_weight_grad / _device_scale (src/bitnet_gpu_dispatch.cpp:284-325;
 * launch_ste_clip_weight_grad(_device_scale)_kernel kernels.cuh:522-527):
 * dW[i] = 0 where |w[i] * (1 / (scale + 1e-8f))| > 1.  The scale is scale_dev[0]
 * when scale_dev is not NULL (device), else `scale` (finite, > 0). */
int nsosx_qat_ste_clip_weight_grad(float* dW, const float* w, int64_t n, float scale,
                                   const float* scale_dev, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NSOSX_H */
