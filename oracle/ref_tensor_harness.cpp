// Test-only C entry points over the reference's own compiled operators, built
// from the reference sources where they lie under /root/reference (oracle/Makefile
// target `ref`; output in oracle/_ref/ only).  Nothing from the reference is
// copied into this tree: this file constructs the reference's types and calls
// their public methods, so the fixtures it produces carry the reference's
// exact arithmetic (sum orders, fma contraction under its -mavx -mfma flags,
// libm calls).
//
// Every function returns 0 on success or -1 when the reference threw; the
// message is then in ref_last_error().
#include <chrono>
#include <cstdint>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

#include "bitlinear.h"
#include "tensor.h"

using nsos::BitLinear;
using nsos::Device;
using nsos::Tensor;

namespace {

thread_local std::string g_error;

Tensor host_tensor(const float* src, std::vector<int> shape) {
  Tensor t(shape, Device::CPU, 0.0f);
  std::memcpy(t.data(), src, sizeof(float) * static_cast<size_t>(t.size));
  return t;
}

void copy_out(const Tensor& t, float* dst) {
  std::memcpy(dst, t.data(), sizeof(float) * static_cast<size_t>(t.size));
}

template <class F>
int guarded(F&& f) {
  try {
    f();
    return 0;
  } catch (const std::exception& e) {
    g_error = e.what();
  } catch (...) {
    g_error = "unknown exception";
  }
  return -1;
}

// A BitLinear [N, K] holding the caller's latent weights, magnitude and bias.
// exact_linear: set_exact_linear_mode(true) (no input RMSNorm, no magnitude),
// as the faithful Mamba-2 projections are configured (src/mamba2.cpp:588-599).
// packed: the CPU packed ternary path (use_reference_path = false,
// src/bitlinear.cpp:690-741); otherwise the float reference path (465-518),
// which quantization-sensitive layers keep.
void configure(BitLinear& bl, const float* w, int N, int K, int exact_linear,
               const float* magnitude, const float* bias, int packed, int training) {
  std::memcpy(bl.weight.data.data(), w, sizeof(float) * static_cast<size_t>(N) * K);
  bl.weight.mark_updated();
  if (magnitude != nullptr) {
    std::memcpy(bl.magnitude.data.data(), magnitude, sizeof(float) * static_cast<size_t>(N));
    bl.magnitude.mark_updated();
  }
  if (bias != nullptr) {
    std::memcpy(bl.bias.data.data(), bias, sizeof(float) * static_cast<size_t>(N));
    bl.bias.mark_updated();
  }
  if (exact_linear) bl.set_exact_linear_mode(true);
  bl.set_training_mode(training != 0);
  bl.set_reference_path(packed == 0);
  bl.repack_weights();
}

}  // namespace

extern "C" {

const char* ref_last_error(void) { return g_error.c_str(); }

// Tensor::rmsnorm (src/tensor.cpp:3455-3492).
int ref_rmsnorm(const float* x, int rows, int cols, float eps, float* out) {
  return guarded([&] { copy_out(host_tensor(x, {rows, cols}).rmsnorm(eps), out); });
}

// Tensor::softmax over the last dimension (src/tensor.cpp:3402-3453).
int ref_softmax(const float* x, int rows, int cols, float* out) {
  return guarded([&] { copy_out(host_tensor(x, {rows, cols}).softmax(-1), out); });
}

// Tensor::silu (src/tensor.cpp:3261-3282).
int ref_silu(const float* x, int64_t n, float* out) {
  return guarded([&] { copy_out(host_tensor(x, {static_cast<int>(n)}).silu(), out); });
}

// Tensor::silu_gate: value * silu(gate) (src/tensor.cpp:3323-3343).
int ref_silu_gate(const float* value, const float* gate, int64_t n, float* out) {
  return guarded([&] {
    const int m = static_cast<int>(n);
    copy_out(Tensor::silu_gate(host_tensor(value, {m}), host_tensor(gate, {m})), out);
  });
}

// Tensor::squared_relu (src/tensor.cpp:3209-3226).
int ref_squared_relu(const float* x, int64_t n, float* out) {
  return guarded([&] { copy_out(host_tensor(x, {static_cast<int>(n)}).squared_relu(), out); });
}

// tensor_abs_mean (src/tensor.cpp:2072-2107).
int ref_abs_mean(const float* w, int64_t n, float* out) {
  return guarded([&] { *out = nsos::tensor_abs_mean(host_tensor(w, {static_cast<int>(n)})); });
}

// Tensor::rmsnorm_backward (src/tensor.cpp:3997-4056), eps 1e-6 as BitLinear uses it.
int ref_rmsnorm_backward(const float* x, const float* grad, const float* x_norm, int rows,
                         int cols, float eps, float* dx) {
  return guarded([&] {
    Tensor xt = host_tensor(x, {rows, cols});
    copy_out(xt.rmsnorm_backward(host_tensor(grad, {rows, cols}),
                                 host_tensor(x_norm, {rows, cols}), eps),
             dx);
  });
}

// BitLinear::forward on the CPU (src/bitlinear.cpp:439-741): packed != 0 runs
// the packed ternary path, else the float reference path.  x [M, K] -> y [M, N].
int ref_bitlinear_forward(const float* w, int N, int K, const float* x, int M, int exact_linear,
                          const float* magnitude, const float* bias, int packed, float* y) {
  return guarded([&] {
    BitLinear bl(K, N, bias != nullptr);
    configure(bl, w, N, K, exact_linear, magnitude, bias, packed, 0);
    copy_out(bl.forward(host_tensor(x, {M, K})), y);
  });
}

// BitLinear::forward then BitLinear::backward in training mode on the packed
// path: the straight-through-estimator backward of src/bitlinear.cpp:1191-1357.
// Outputs y [M, N], dx [M, K], dW [N, K], dmag [N] (NULL in exact-linear
// mode), dbias [N] (NULL without bias).
int ref_bitlinear_packed_backward(const float* w, int N, int K, const float* x, int M,
                                  int exact_linear, const float* magnitude, const float* bias,
                                  const float* grad, float* y, float* dx, float* dW,
                                  float* dmag, float* dbias) {
  return guarded([&] {
    BitLinear bl(K, N, bias != nullptr);
    configure(bl, w, N, K, exact_linear, magnitude, bias, 1, 1);
    copy_out(bl.forward(host_tensor(x, {M, K})), y);
    copy_out(bl.backward(host_tensor(grad, {M, N})), dx);
    copy_out(bl.weight.grad, dW);
    if (dmag != nullptr) copy_out(bl.magnitude.grad, dmag);
    if (dbias != nullptr) copy_out(bl.bias.grad, dbias);
  });
}

// Seconds per BitLinear::forward on the CPU packed path (RMS_PERI + magnitude,
// or exact-linear), over `reps` calls on one configured layer (packing is done
// once, outside the timed loop): the reference's own CPU hot path, for the
// CPU baseline.  y receives the last call's output.
int ref_bitlinear_time_forward(const float* w, int N, int K, const float* x, int M,
                               int exact_linear, int reps, float* y, double* seconds) {
  return guarded([&] {
    BitLinear bl(K, N, false);
    configure(bl, w, N, K, exact_linear, nullptr, nullptr, 1, 0);
    Tensor in = host_tensor(x, {M, K});
    Tensor out = bl.forward(in);  // warm (first-call allocations)
    const auto t0 = std::chrono::steady_clock::now();
    for (int r = 0; r < reps; ++r) out = bl.forward(in);
    const auto t1 = std::chrono::steady_clock::now();
    *seconds = std::chrono::duration<double>(t1 - t0).count() / (reps > 0 ? reps : 1);
    copy_out(out, y);
  });
}

}  // extern "C"
