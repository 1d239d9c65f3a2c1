/*
 * nsos_oracle.h -- CPU restatement of the reference's hybrid-layer hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links, loads or
 * calls this code: it is the checker that tests/, __graft_entry__.smoke() and
 * the cpu_baseline leg of bench.py compare the HIP path against.
 *
 * Every function cites the reference file:line it restates (paths are under
 * OXN/nsos/ of vitorGgC569/reimagined).  Layouts are plain row-major arrays.
 */
#ifndef NSOS_ORACLE_H
#define NSOS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- BitLinear weights -------------------------------------------------- */
float orc_absmean(const float* w, int64_t n);
float orc_weight_scale(const float* w, int64_t n);
void orc_ternary_codes(const float* w, int64_t n, float weight_scale, int8_t* codes);
void orc_pack_codes(const int8_t* codes, int64_t n, uint8_t* packed);
void orc_unpack_codes(const uint8_t* packed, int64_t n, int8_t* codes);
int64_t orc_find_reserved_code(const uint8_t* packed, int64_t n);
void orc_row_sums(const int8_t* w, int rows, int cols, int32_t* sums);

/* ---- BitLinear activations and GEMM -------------------------------------- */
float orc_q_max(int bits);
void orc_rmsnorm(const float* x, int rows, int cols, float eps, float* out);
void orc_quantize_act(const float* x, int rows, int cols, int bits, int8_t* q,
                      float* act_scale);
void orc_gemm_i8(const int8_t* q, const int8_t* w, int M, int K, int N, int32_t* acc);
void orc_dequant(const int32_t* acc, const float* act_scale, float weight_scale,
                 const float* magnitude, const float* bias, int M, int N, float* y);
void orc_bitlinear_forward(const float* x, int M, int K, int N, const uint8_t* packed,
                           float weight_scale, int bits, int rms_input,
                           const float* magnitude, const float* bias, float* y,
                           int8_t* q_out, float* act_scale_out, int32_t* acc_out);

/* ---- elementwise ---------------------------------------------------------- */
float orc_silu(float v);
void orc_conv_step(const float* x, int rows, int channels, const float* weight,
                   const float* bias, int width, float* ring, int apply_silu, float* out);
void orc_rmsnorm_gated(const float* y, const float* z, const float* gamma, int rows, int cols,
                       float eps, float* out);

/* Quantization-aware training: fake-quant forward and the STE clip
 * (OXN/nsos/src/bitnet_gpu_dispatch.cpp:193-325). */
void orc_qat_fake_quant_ternary(const float* w, int64_t n, float scale, float* out);
float orc_qat_fake_quant_ternary_absmean(const float* w, int64_t n, float* out);
void orc_qat_fake_quant_activations(const float* x, int M, int K, int bits, float* out);
void orc_qat_ste_clip(float* dW, const float* w, int64_t n, float scale);
float orc_softplus(float v);
void orc_squared_relu(const float* x, int64_t n, float* out);

/* ---- Mamba selective scan -------------------------------------------------- */
void orc_decay_terms(float dt_raw, float a_log, float* delta, float* decay);
void orc_conv1d_causal(const float* in, const float* weight, const float* bias,
                       const int32_t* cu_seqlens, int num_seqs, int channels,
                       int width, int apply_silu, float* out);
void orc_selective_scan(const float* x, const float* dt, const float* a_log,
                        int a_per_state, const float* B, const float* C,
                        const float* Dskip, const float* z, const int32_t* cu_seqlens,
                        int num_seqs, int H, int P, int N, int G,
                        const float* initial_state, float* y, float* final_state,
                        int gate_silu);
void orc_scan_step(const float* x, const float* dt, const float* a_log, int a_per_state,
                   const float* B, const float* C, const float* Dskip, const float* z,
                   int rows, int H, int P, int N, int G, float* state, float* y,
                   int gate_silu);

/* ---- BitLinear float path and packed STE backward ------------------------- */
void orc_rmsnorm_backward(const float* x, const float* g, const float* y, int rows, int cols,
                          float eps, float* dx);
void orc_linear_f32(const float* x, int M, int K, int N, const float* w, int rms_input,
                    const float* magnitude, const float* bias, float* y);
void orc_bitlinear_ste_backward(const float* x, const int8_t* q, const float* as,
                                const float* w, const int8_t* codes, float ws, int M, int K,
                                int N, int rms_input, const float* magnitude, const float* grad,
                                float* dx, float* dW, float* dmag, float* dbias);

/* ---- MoE routing / dispatch ---------------------------------------------- */
void orc_softmax_rows(const float* logits, int rows, int cols, float* probs);
void orc_topk_mask(float* weights, int rows, int experts, int k, int32_t* selected);
void orc_zero_invalid_rows(float* weights, int32_t* selected, const uint8_t* valid, int rows,
                           int experts, int k);
void orc_expert_loads(const float* weights, const uint8_t* valid, int rows, int experts,
                      float* loads);
void orc_moe_dispatch_sel(const int32_t* sel, int rows, int experts, int k, int32_t* counts,
                          int32_t* offsets, int32_t* perm);
void orc_moe_dispatch(const float* weights, int rows, int experts, int k,
                      int32_t* counts, int32_t* offsets, int32_t* perm);
void orc_moe_combine(const float* expert_out, const int32_t* perm, const int32_t* offsets,
                     const float* weights, int rows, int experts, int dim, float* out);

#ifdef __cplusplus
}
#endif

#endif
