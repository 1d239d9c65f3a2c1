// nsosx.hpp -- C++ host mirror of the reference operator API over the C ABI
// (include/nsosx.h), for C++ callers of the hot path: the role the reference's
// BitLinear / MoERouter / Mamba scan entry points play for OXN/nsos
// (include/bitlinear.h, include/jamba.h, include/cuda/mamba_kernels.cuh).
//
// Header-only; needs the HIP runtime API (hipMalloc, hipMemcpy) and
// libnsosx.so.  Errors follow the reference: rejected arguments throw
// std::invalid_argument, size overflows std::overflow_error, runtime failures
// std::runtime_error, each with the library's message.  Work is enqueued on
// the given stream without synchronising; objects own their device buffers.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "nsosx.h"

namespace nsosx {

inline void check(int rc, const char* what) {
    if (rc == NSOSX_OK) return;
    const std::string msg = std::string(what) + ": " + nsosx_last_error();
    if (rc == NSOSX_ERR_INVALID || rc == NSOSX_ERR_RESERVED) throw std::invalid_argument(msg);
    if (rc == NSOSX_ERR_OVERFLOW) throw std::overflow_error(msg);
    throw std::runtime_error(msg);
}

inline void check_hip(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// Owning device allocation (the role of the reference Tensor's device storage).
class DeviceBuffer {
  public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t bytes) { resize(bytes); }
    ~DeviceBuffer() { release(); }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&& o) noexcept : p_(o.p_), bytes_(o.bytes_) { o.p_ = nullptr; o.bytes_ = 0; }
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
        if (this != &o) {
            release();
            p_ = o.p_; bytes_ = o.bytes_;
            o.p_ = nullptr; o.bytes_ = 0;
        }
        return *this;
    }
    // Grows (never shrinks) the allocation; the contents are not kept.
    void reserve(size_t bytes) {
        if (bytes > bytes_) resize(bytes);
    }
    void resize(size_t bytes) {
        release();
        if (bytes) check_hip(hipMalloc(&p_, bytes), "hipMalloc");
        bytes_ = bytes;
    }
    template <class T>
    void upload(const std::vector<T>& v) {
        resize(v.size() * sizeof(T));
        if (bytes_) check_hip(hipMemcpy(p_, v.data(), bytes_, hipMemcpyHostToDevice), "upload");
    }
    template <class T>
    std::vector<T> download(size_t count) const {
        std::vector<T> v(count);
        if (count) check_hip(hipMemcpy(v.data(), p_, count * sizeof(T), hipMemcpyDeviceToHost), "download");
        return v;
    }
    void* data() const { return p_; }
    template <class T>
    T* as() const { return static_cast<T*>(p_); }
    size_t bytes() const { return bytes_; }

  private:
    void release() {
        if (p_) (void)hipFree(p_);
        p_ = nullptr;
        bytes_ = 0;
    }
    void* p_ = nullptr;
    size_t bytes_ = 0;
};

// The packed fields of BitLinearPackedState (include/bitlinear.h:37-47).
struct PackedState {
    int in_features = 0;
    int out_features = 0;
    float weight_scale = 1.0f;
    std::vector<uint32_t> packed_weights;   // reference layout, [out * in / 16]
    std::vector<float> magnitude;           // [out] or empty (unit)
    std::vector<float> bias;                // [out] or empty
};

// BitLinear (include/bitlinear.h, src/bitlinear.cpp): a ternary projection on
// the packed path (RMS_PERI + int8 activations + ternary GEMM + magnitude/bias),
// or, for quantization-sensitive layers, the float path (fp32 weights).
class BitLinear {
  public:
    BitLinear(int in_features, int out_features, bool use_bias)
        : in_(in_features), out_(out_features), use_bias_(use_bias) {
        if (in_features <= 0 || out_features <= 0)
            throw std::invalid_argument("BitLinear features must be positive");
    }

    // BitLinear::quantize_weights + pack_weights on the latent fp32 weights [out, in].
    void set_weights(const std::vector<float>& w) {
        if (w.size() != (size_t)in_ * out_) throw std::invalid_argument("BitLinear weights: size");
        std::vector<uint32_t> packed(in_ % 16 == 0 ? (size_t)out_ * in_ / 16 : 0);
        float ws = 0.0f;
        check(nsosx_pack_ternary(w.data(), out_, in_, packed.data(), &ws), "pack_ternary");
        upload_packed(packed, ws);
        latent_.upload(w);  // the float path and the STE clip use the latent weights
    }

    // BitLinear::import_packed_state: rejects the reserved code 3 (src/bitlinear.cpp:876-885).
    void import_packed_state(const PackedState& s) {
        if (s.in_features != in_ || s.out_features != out_ ||
            s.packed_weights.size() != (size_t)in_ * out_ / 16)
            throw std::invalid_argument("BitLinear::import_packed_state: shape mismatch");
        upload_packed(s.packed_weights, s.weight_scale);
        DeviceBuffer bad(sizeof(int64_t));
        check(nsosx_find_reserved_code(packed_.as<uint32_t>(), (int64_t)in_ * out_,
                                       bad.as<int64_t>(), nullptr), "find_reserved_code");
        const int64_t first = bad.download<int64_t>(1)[0];
        if (first >= 0)
            throw std::invalid_argument("BitLinear::import_packed_state: reserved code 3 at " +
                                        std::to_string(first));
        if (!s.magnitude.empty()) set_magnitude(s.magnitude);
        if (!s.bias.empty()) set_bias(s.bias);
    }

    PackedState export_packed_state() const {
        PackedState s;
        s.in_features = in_;
        s.out_features = out_;
        s.weight_scale = weight_scale_;
        s.packed_weights = packed_.download<uint32_t>((size_t)in_ * out_ / 16);
        if (magnitude_.bytes()) s.magnitude = magnitude_.download<float>(out_);
        if (bias_.bytes()) s.bias = bias_.download<float>(out_);
        return s;
    }

    void set_magnitude(const std::vector<float>& m) {
        if (m.size() != (size_t)out_) throw std::invalid_argument("BitLinear magnitude: size");
        magnitude_.upload(m);
    }
    void set_bias(const std::vector<float>& b) {
        if (!use_bias_) throw std::invalid_argument("BitLinear built without bias");
        if (b.size() != (size_t)out_) throw std::invalid_argument("BitLinear bias: size");
        bias_.upload(b);
    }
    // set_exact_linear_mode (include/bitlinear.h:99-108): no input RMSNorm, no magnitude.
    void set_exact_linear_mode(bool on) { exact_linear_ = on; }
    // set_quantization_sensitive: the float path with the latent weights.
    void set_quantization_sensitive(bool on) { sensitive_ = on; }
    void set_precision_mode(int bits) {
        if (bits < 2 || bits > 8) throw std::invalid_argument("BitLinear precision must be in [2, 8]");
        bits_ = bits;
    }

    // BitLinear::forward for M rows: x [M, in] (x_dtype) -> y [M, out] (y_dtype), device.
    void forward(const void* x, int x_dtype, int M, void* y, int y_dtype,
                 hipStream_t stream = nullptr) {
        if (!packed_.bytes()) throw std::runtime_error("BitLinear::forward before set_weights");
        const int rms = exact_linear_ ? 0 : 1;
        const float* mag = exact_linear_ || !magnitude_.bytes() ? nullptr : magnitude_.as<float>();
        const float* bias = bias_.bytes() ? bias_.as<float>() : nullptr;
        rms_ws_.reserve((size_t)M * sizeof(float));
        if (sensitive_) {
            check(nsosx_linear_f32(x, x_dtype, M, in_, latent_.as<float>(), out_, rms, mag, bias,
                                   y, y_dtype, rms_ws_.as<float>(), stream),
                  "BitLinear::forward (float path)");
            return;
        }
        q_ws_.reserve((size_t)M * in_);
        scale_ws_.reserve((size_t)M * sizeof(float));
        check(nsosx_quantize_act_i8(x, x_dtype, M, in_, bits_, rms, q_ws_.as<int8_t>(),
                                    scale_ws_.as<float>(), rms_ws_.as<float>(), stream),
              "BitLinear::forward (quantize)");
        if (M > 128 && packed_mfma_.bytes())
            check(nsosx_ternary_gemm_mfma(q_ws_.as<int8_t>(), scale_ws_.as<float>(),
                                          packed_mfma_.as<uint32_t>(), weight_scale_, M, in_,
                                          out_, mag, bias, y, y_dtype, nullptr, stream),
                  "BitLinear::forward (GEMM)");
        else
            check(nsosx_ternary_gemm(q_ws_.as<int8_t>(), scale_ws_.as<float>(),
                                     packed_.as<uint32_t>(), weight_scale_, M, in_, out_, mag,
                                     bias, y, y_dtype, nullptr, stream),
                  "BitLinear::forward (GEMM)");
    }

    int input_features() const { return in_; }
    int output_features() const { return out_; }
    float weight_scale() const { return weight_scale_; }

  private:
    void upload_packed(const std::vector<uint32_t>& packed, float ws) {
        packed_.upload(packed);
        weight_scale_ = ws;
        if (in_ % 128 == 0) {
            packed_mfma_.resize(packed.size() * sizeof(uint32_t));
            check(nsosx_pack_mfma_layout(packed_.as<uint32_t>(), (int64_t)packed.size(),
                                         packed_mfma_.as<uint32_t>(), nullptr),
                  "pack_mfma_layout");
            check_hip(hipDeviceSynchronize(), "pack_mfma_layout");
        }
    }

    int in_, out_;
    bool use_bias_;
    bool exact_linear_ = false;
    bool sensitive_ = false;
    int bits_ = 8;
    float weight_scale_ = 1.0f;
    DeviceBuffer packed_, packed_mfma_, latent_, magnitude_, bias_;
    DeviceBuffer q_ws_, scale_ws_, rms_ws_;
};

// MoERouter::forward(x, valid_rows) from logits (src/jamba.cpp:8140-8319) with the
// ordered dispatch of forward_moe: device outputs, owned by the router.
class MoERouter {
  public:
    MoERouter(int num_experts, int top_k) : e_(num_experts), k_(top_k) {
        if (num_experts <= 0 || top_k <= 0 || top_k > num_experts)
            throw std::invalid_argument("MoERouter requires num_experts > 0, 0 < top_k <= num_experts");
    }
    struct Routing {
        const float* weights;     // [rows, E]
        const int32_t* selected;  // [rows, k] (-1 on padding rows)
        const int32_t* counts;    // [E]
        const int32_t* offsets;   // [E + 1]
        const int32_t* perm;      // [rows * k] (the first offsets[E] entries)
        const int32_t* slot_of;   // [rows, k] (-1 on padding rows)
        const float* loads;       // [E] (expert_loads) when asked for, else nullptr
    };
    // valid_rows: the reference's host mask, empty (every row valid) or one 0 / 1 per
    // row, validated as MoERouter::forward does (src/jamba.cpp:8145-8153) and uploaded
    // on `stream`.  want_loads: also the per-expert loads.
    Routing route(const float* logits, int rows, hipStream_t stream = nullptr,
                  const std::vector<uint8_t>& valid_rows = {}, bool want_loads = false) {
        if (!valid_rows.empty()) {
            if (valid_rows.size() != static_cast<size_t>(rows))
                throw std::invalid_argument("MoERouter valid-row mask size mismatch");
            for (uint8_t v : valid_rows)
                if (v > 1) throw std::invalid_argument("MoERouter valid-row mask must contain only 0 or 1");
            mask_.reserve((size_t)rows);
            check_hip(hipMemcpyAsync(mask_.data(), valid_rows.data(), (size_t)rows,
                                     hipMemcpyHostToDevice, stream),
                      "MoE valid-row mask upload");
        }
        weights_.reserve((size_t)rows * e_ * 4);
        selected_.reserve((size_t)rows * k_ * 4);
        counts_.reserve((size_t)e_ * 4);
        offsets_.reserve((size_t)(e_ + 1) * 4);
        perm_.reserve((size_t)rows * k_ * 4);
        slot_of_.reserve((size_t)rows * k_ * 4);
        if (want_loads) loads_.reserve((size_t)e_ * 4);
        ws_.reserve((size_t)nsosx_moe_route_workspace(rows, e_) * 4 + 4);
        float* loads = want_loads ? loads_.as<float>() : nullptr;
        check(nsosx_moe_route(logits, valid_rows.empty() ? nullptr : mask_.as<uint8_t>(), rows,
                              e_, k_, weights_.as<float>(), selected_.as<int32_t>(),
                              counts_.as<int32_t>(), offsets_.as<int32_t>(), perm_.as<int32_t>(),
                              slot_of_.as<int32_t>(), loads, ws_.as<int32_t>(), stream),
              "MoERouter::forward");
        return {weights_.as<float>(), selected_.as<int32_t>(), counts_.as<int32_t>(),
                offsets_.as<int32_t>(), perm_.as<int32_t>(), slot_of_.as<int32_t>(), loads};
    }

  private:
    int e_, k_;
    DeviceBuffer weights_, selected_, counts_, offsets_, perm_, slot_of_, loads_, mask_, ws_;
};

// The Mamba selective scan over a packed ragged batch (src/mamba2.cpp:2602-2675)
// through the planned entry point: the workspace is owned here and grown on demand.
class SelectiveScan {
  public:
    struct Shape { int H, P, N, G; };
    // x (conv input when conv_w != nullptr), dt, B, C, z in act_dtype; see
    // nsosx_scan_fwd_planned for the layouts.  chunk_tokens: -1 auto, 0 never, > 0 fixed.
    void forward(const void* x, int64_t x_stride, const float* conv_w, const float* conv_b,
                 int conv_width, const void* dt, const float* A_log, bool a_per_state,
                 const void* B, const void* C, const float* D, const void* z, int64_t z_stride,
                 const int32_t* cu_seqlens, int num_seqs, int total_tokens, Shape s, int act_dtype,
                 const float* initial_state, float* final_state, void* y, int chunk_tokens = -1,
                 hipStream_t stream = nullptr) {
        const int64_t bytes = nsosx_scan_fwd_workspace(num_seqs, total_tokens, s.H, s.P, s.N,
                                                       chunk_tokens);
        ws_.reserve((size_t)bytes + 256);
        check(nsosx_scan_fwd_planned(x, x_stride, conv_w, conv_b, conv_width, dt, A_log,
                                     a_per_state ? 1 : 0, B, C, D, z, z_stride, cu_seqlens,
                                     num_seqs, total_tokens, s.H, s.P, s.N, s.G, act_dtype,
                                     initial_state, final_state, y, chunk_tokens, ws_.data(),
                                     stream),
              "selective scan");
    }

  private:
    DeviceBuffer ws_;
};

}  // namespace nsosx
