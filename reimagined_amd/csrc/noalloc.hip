// nsosx_bitlinear_forward_noalloc: the BitLinear forward with its activation
// workspace (int8 codes, act_scale, RMS inverse) taken from a library-owned
// device array instead of caller buffers, for callers that cannot allocate
// (code under HIP graph capture, serving loops that forbid hipMalloc).
//
// The array is a file-scope __device__ symbol: every GPU the library runs on
// holds its own copy at its own address from module load until the process
// ends.  Host code never passes the symbol's name to a kernel (on the host it
// is only a stand-in, not a device address); the device address is looked up
// once per device with hipGetSymbolAddress, on the first call made on that
// device outside HIP graph capture, and kept in g_scratch_ptr.  A first call
// on a device whose stream is capturing is refused (the lookup may load the
// code object, which has no place inside a capture): run the entry once
// eagerly on each device, then capture it.
#include "common.hpp"

#include <mutex>

namespace nsosx {

// Upper bound of the workspace: M*K code bytes (rounded up to 256) plus two
// float vectors of M (each rounded up to 256).
constexpr int64_t kNoallocScratchBytes = int64_t(8) << 20;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

static void* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

static int64_t round256(int64_t v) { return (v + 255) & ~int64_t(255); }

// Device address of this device's scratch array (looked up on the first call on
// each device, with that device current and its stream not capturing).
static int scratch_for_current_device(hipStream_t st, unsigned char** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return fail(NSOSX_ERR_LAUNCH, std::string("bitlinear_forward_noalloc: hipGetDevice: ") +
                                          hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices)
        return fail(NSOSX_ERR_INVALID, "bitlinear_forward_noalloc: device index out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(st, &cs);
        if (e != hipSuccess || cs != hipStreamCaptureStatusNone)
            return fail(NSOSX_ERR_INVALID,
                        "bitlinear_forward_noalloc: the first call on a device must be made "
                        "outside HIP graph capture (it looks up the scratch array's address)");
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(NSOSX_ERR_LAUNCH,
                        std::string("bitlinear_forward_noalloc: hipGetSymbolAddress: ") +
                            hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = static_cast<unsigned char*>(g_scratch_ptr[dev]);
    return NSOSX_OK;
}

}  // namespace nsosx

using namespace nsosx;

extern "C" int64_t nsosx_bitlinear_forward_noalloc_max_bytes(void) {
    return kNoallocScratchBytes;
}

extern "C" int nsosx_bitlinear_forward_noalloc(const void* x, int x_dtype,
                                               const uint32_t* packed, float weight_scale, int M,
                                               int K, int N, int precision_bits, int rms_input,
                                               const float* magnitude, const float* bias, void* y,
                                               int y_dtype, void* stream) {
    if (M <= 0 || K <= 0) return fail(NSOSX_ERR_INVALID, "bitlinear_forward_noalloc: empty shape");
    const int64_t q_bytes = round256((int64_t)M * K);
    const int64_t v_bytes = round256((int64_t)M * (int64_t)sizeof(float));
    if (q_bytes + 2 * v_bytes > kNoallocScratchBytes)
        return fail(NSOSX_ERR_OVERFLOW,
                    "bitlinear_forward_noalloc: M*K + 8*M bytes of workspace exceed the "
                    "library's 8 MiB scratch; use nsosx_bitlinear_forward with caller buffers");
    unsigned char* base = nullptr;
    int rc = scratch_for_current_device(static_cast<hipStream_t>(stream), &base);
    if (rc) return rc;
    int8_t* q = reinterpret_cast<int8_t*>(base);
    float* scale = reinterpret_cast<float*>(base + q_bytes);
    float* rms = reinterpret_cast<float*>(base + q_bytes + v_bytes);
    return nsosx_bitlinear_forward(x, x_dtype, packed, weight_scale, M, K, N, precision_bits,
                                   rms_input, magnitude, bias, y, y_dtype, q, scale,
                                   rms_input ? rms : nullptr, stream);
}
