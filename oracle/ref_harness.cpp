// Test-only harness around the reference's own AVX2 activation-quantization
// helpers, compiled from OXN/nsos/src/bitlinear_quantize_avx2.cpp where it
// lies under /root/reference (see oracle/Makefile target `ref`).  Output goes
// to oracle/_ref/ only; nothing from the reference is copied into this tree.
//
// The per-row driver below restates the three lines of
// BitLinear::quantize_activations_bitnet that call those helpers
// (OXN/nsos/src/bitlinear.cpp:271-277); the helpers themselves are the
// reference's compiled code.
#include <cmath>
#include <cstdint>

namespace nsos {
float bitlinear_row_max_abs_avx2(const float* row_ptr, int K);
void bitlinear_row_scale_round_avx2(float* dst, const float* src, int K, float scale);
int32_t bitlinear_row_sum_i8_avx2(const int8_t* row_ptr, int cols);
}  // namespace nsos

extern "C" {

// codes: float round(x*scale) as the reference stores them; scales: act_scale.
void ref_quantize_rows(const float* x, int rows, int cols, int bits, float* codes,
                       float* scales) {
  float q_max = 127.0f;
  if (bits <= 2) q_max = 1.0f;
  else q_max = std::pow(2.0f, bits - 1) - 1.0f;
  for (int i = 0; i < rows; ++i) {
    const float* row = x + static_cast<long>(i) * cols;
    const float max_val = nsos::bitlinear_row_max_abs_avx2(row, cols);
    const float scale = q_max / (max_val + 1e-8f);
    scales[i] = (max_val + 1e-8f) / q_max;
    nsos::bitlinear_row_scale_round_avx2(codes + static_cast<long>(i) * cols, row, cols, scale);
  }
}

int32_t ref_row_sum_i8(const int8_t* row, int cols) {
  return nsos::bitlinear_row_sum_i8_avx2(row, cols);
}

}  // extern "C"
