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
#include <stdexcept>
#include <utility>
#include <string>
#include <vector>

#include "bitlinear.h"
#include "mamba2.h"
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

// Mamba2SSD::forward on the faithful Mamba-2 path (src/mamba2.cpp:2360-2681), CPU.
// The block is built with MambaConfig{faithful_mamba2, expand, head_dim,
// n_groups, conv_kernel}; every parameter is overwritten with the caller's
// (w_x, w_z [inner, d]; w_B, w_C [G*N, d]; w_dt [H, d]; dt_bias [H]; w_out
// [d, inner]; conv_w [inner + 2 G N, K]; conv_b [inner + 2 G N]; a_log, d_skip
// [H]; norm_w [inner]).  packed != 0 puts the non-sensitive projections (x, z,
// out_proj) on the packed ternary path, as quantized deployment runs them; B,
// C and dt stay on the float path (quantization-sensitive).  u [batch, seq, d]
// -> out [batch, seq, d].
int ref_mamba2_faithful_forward(int d_model, int d_state, int expand, int head_dim,
                                int n_groups, int conv_kernel, const float* w_x,
                                const float* w_z, const float* w_B, const float* w_C,
                                const float* w_dt, const float* dt_bias, const float* w_out,
                                const float* conv_w, const float* conv_b, const float* a_log,
                                const float* d_skip, const float* norm_w, int packed,
                                const float* u, int batch, int seq, float* out) {
  return guarded([&] {
    nsos::MambaConfig cfg;
    cfg.faithful_mamba2 = true;
    cfg.expand = expand;
    cfg.head_dim = head_dim;
    cfg.n_groups = n_groups;
    cfg.conv_kernel = conv_kernel;
    nsos::Mamba2SSD blk(d_model, d_state, 1, cfg);
    blk.set_training_mode(false);
    const int inner = d_model * expand;
    const int heads = inner / head_dim;
    const int gs = n_groups * d_state;
    const int conv_dim = inner + 2 * gs;
    auto fill = [](nsos::Parameter* p, const float* src, size_t n) {
      if (static_cast<size_t>(p->data.size) != n)
        throw std::runtime_error("parameter " + p->name + " has an unexpected size");
      std::memcpy(p->data.data(), src, sizeof(float) * n);
      p->mark_updated();
    };
    const std::vector<std::pair<std::string, std::pair<const float*, size_t>>> want = {
        {"x_proj.weight", {w_x, (size_t)inner * d_model}},
        {"z_proj.weight", {w_z, (size_t)inner * d_model}},
        {"B_proj.weight", {w_B, (size_t)gs * d_model}},
        {"C_proj.weight", {w_C, (size_t)gs * d_model}},
        {"dt_proj.weight", {w_dt, (size_t)heads * d_model}},
        {"dt_proj.bias", {dt_bias, (size_t)heads}},
        {"out_proj.weight", {w_out, (size_t)d_model * inner}},
        {"conv1d_weight", {conv_w, (size_t)conv_dim * conv_kernel}},
        {"conv1d_bias", {conv_b, (size_t)conv_dim}},
        {"norm.weight", {norm_w, (size_t)inner}},
        {"A", {a_log, (size_t)heads}},
        {"D", {d_skip, (size_t)heads}},
    };
    std::vector<nsos::Parameter*> params = blk.parameters();
    for (const auto& [name, src] : want) {
      nsos::Parameter* hit = nullptr;
      for (nsos::Parameter* p : params)
        if (p->name == name) hit = p;
      if (!hit) throw std::runtime_error("no parameter named " + name);
      fill(hit, src.first, src.second);
    }
    std::vector<BitLinear*> layers;
    blk.collect_bitlinear_layers(layers);  // x, z, B, C, dt, out_proj
    for (size_t i = 0; i < layers.size(); ++i) {
      BitLinear* bl = layers[i];
      bl->set_training_mode(false);
      const bool sensitive = i >= 2 && i <= 4;
      bl->set_reference_path(!(packed && !sensitive));
      bl->repack_weights();
    }
    Tensor in = host_tensor(u, {batch, seq, d_model});
    copy_out(blk.forward(in), out);
  });
}

}  // extern "C"
