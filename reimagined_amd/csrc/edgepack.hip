// Host-side reader of the reference's edge linear pack ("DGE1"), the on-disk
// format BitLinear layers are shipped in (JambaModel::save_edge_linear_pack /
// load_edge_linear_pack, OXN/nsos/src/jamba.cpp:1325-1620; helpers 504-616).
//
//   u32 magic 0x31454744 ("DGE1"), u32 version (3, or the legacy 2),
//   u32 layer count, then per layer:
//     u8 sensitive, i32 in_features, i32 out_features, u8 use_bias,
//     f32 weight_scale,
//     vector<u32> packed_weights   (u64 count, then the words)
//     vector<f32> magnitude, bias, flat_alpha, flat_beta
//     vector<f32> fp32 weights     (sensitive layers only)
//   version 3 appends a trailer: u32 0x33494745 ("EGI3"), u64 payload bytes,
//   64 ASCII hex digits of the payload's SHA-256.
//
// Parsing is zero-copy: every vector is returned as a byte offset into the
// caller's buffer, so the packed words can be uploaded straight to the device
// in the format the GEMM/GEMV kernels read.  SHA-256 follows FIPS 180-4; its
// round constants and initial hash are derived here from the primes the
// standard defines them by (fractional bits of cube / square roots).
#include "common.hpp"

#include <cmath>
#include <cstring>

namespace nsosx {
namespace {

struct Sha256 {
    uint32_t k[64];
    uint32_t h0[8];

    Sha256() {
        // first 64 primes; k = first 32 fractional bits of their cube roots,
        // h0 = first 32 fractional bits of the square roots of the first 8
        int primes[64];
        int n = 0;
        for (int c = 2; n < 64; ++c) {
            bool prime = true;
            for (int d = 2; d * d <= c; ++d)
                if (c % d == 0) { prime = false; break; }
            if (prime) primes[n++] = c;
        }
        for (int i = 0; i < 64; ++i) k[i] = frac32(cbrtl(static_cast<long double>(primes[i])));
        for (int i = 0; i < 8; ++i) h0[i] = frac32(sqrtl(static_cast<long double>(primes[i])));
    }

    static uint32_t frac32(long double v) {
        const long double f = v - floorl(v);
        return static_cast<uint32_t>(floorl(f * 4294967296.0L));
    }

    static uint32_t rotr(uint32_t x, int s) { return (x >> s) | (x << (32 - s)); }

    void block(uint32_t h[8], const uint8_t* p) const {
        uint32_t w[64];
        for (int i = 0; i < 16; ++i)
            w[i] = (uint32_t)p[4 * i] << 24 | (uint32_t)p[4 * i + 1] << 16 |
                   (uint32_t)p[4 * i + 2] << 8 | (uint32_t)p[4 * i + 3];
        for (int i = 16; i < 64; ++i) {
            const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
            const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
            w[i] = w[i - 16] + s0 + w[i - 7] + s1;
        }
        uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
        for (int i = 0; i < 64; ++i) {
            const uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
            const uint32_t ch = (e & f) ^ (~e & g);
            const uint32_t t1 = hh + S1 + ch + k[i] + w[i];
            const uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
            const uint32_t maj = (a & b) ^ (a & c) ^ (b & c);
            const uint32_t t2 = S0 + maj;
            hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
        }
        h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
    }

    void hex(const uint8_t* data, uint64_t size, char out[65]) const {
        uint32_t h[8];
        std::memcpy(h, h0, sizeof(h));
        uint64_t off = 0;
        for (; off + 64 <= size; off += 64) block(h, data + off);
        // padding: 0x80, zeros, then the bit length big-endian, to a 64-byte multiple
        uint8_t tail[128] = {0};
        const uint64_t rem = size - off;
        std::memcpy(tail, data + off, rem);
        tail[rem] = 0x80;
        const uint64_t nblk = rem + 9 <= 64 ? 1 : 2;
        const uint64_t bits = size * 8;
        for (int i = 0; i < 8; ++i) tail[nblk * 64 - 1 - i] = static_cast<uint8_t>(bits >> (8 * i));
        for (uint64_t b = 0; b < nblk; ++b) block(h, tail + 64 * b);
        static const char* digits = "0123456789abcdef";
        for (int i = 0; i < 8; ++i)
            for (int j = 0; j < 8; ++j) out[8 * i + j] = digits[(h[i] >> (28 - 4 * j)) & 15];
        out[64] = '\0';
    }
};

const Sha256& sha256() {
    static const Sha256 s;
    return s;
}

constexpr uint32_t kEdgeMagic = 0x31454744u;      // "DGE1"
constexpr uint32_t kEdgeTrailerMagic = 0x33494745u;  // "EGI3"
constexpr uint64_t kEdgeTrailerBytes = 4 + 8 + 64;

struct Reader {
    const uint8_t* p;
    uint64_t size, pos;
    bool ok = true;
    template <typename T>
    T pod() {
        T v{};
        if (pos + sizeof(T) > size) { ok = false; return v; }
        std::memcpy(&v, p + pos, sizeof(T));
        pos += sizeof(T);
        return v;
    }
    // vector<T>: u64 count (must equal `need`), then count elements; returns the offset
    uint64_t vec(uint64_t need, uint64_t elem, bool& count_ok) {
        const uint64_t count = pod<uint64_t>();
        count_ok = ok && count == need;
        const uint64_t off = pos;
        if (!count_ok || count > (size - pos) / elem) { ok = false; return 0; }
        pos += count * elem;
        return off;
    }
};

bool all_finite(const uint8_t* base, uint64_t off, uint64_t count) {
    for (uint64_t i = 0; i < count; ++i) {
        float v;
        std::memcpy(&v, base + off + 4 * i, 4);
        if (!std::isfinite(v)) return false;
    }
    return true;
}

}  // namespace
}  // namespace nsosx

using namespace nsosx;

extern "C" int nsosx_sha256_hex(const uint8_t* data, uint64_t size, char* hex_out) {
    if ((!data && size) || !hex_out) return fail(NSOSX_ERR_INVALID, "sha256: null pointer");
    sha256().hex(data, size, hex_out);
    return NSOSX_OK;
}

extern "C" int nsosx_edge_pack_parse(const uint8_t* data, uint64_t size, nsosx_edge_layer* layers,
                                     int max_layers, int* num_layers, uint32_t* version_out) {
    if (!data || !num_layers || (max_layers > 0 && !layers))
        return fail(NSOSX_ERR_INVALID, "edge_pack: null pointer");
    *num_layers = 0;
    Reader rd{data, size, 0};
    const uint32_t magic = rd.pod<uint32_t>();
    if (!rd.ok || magic != kEdgeMagic) return fail(NSOSX_ERR_INVALID, "edge_pack: invalid header");
    const uint32_t version = rd.pod<uint32_t>();
    if (!rd.ok || (version != 2 && version != 3))
        return fail(NSOSX_ERR_INVALID, "edge_pack: unsupported version");
    if (version_out) *version_out = version;
    uint64_t payload = size;
    if (version == 3) {
        if (size < 12 + kEdgeTrailerBytes)
            return fail(NSOSX_ERR_INVALID, "edge_pack: too small for its integrity trailer");
        Reader tr{data, size, size - kEdgeTrailerBytes};
        const uint32_t tmagic = tr.pod<uint32_t>();
        const uint64_t pbytes = tr.pod<uint64_t>();
        if (tmagic != kEdgeTrailerMagic || pbytes != size - kEdgeTrailerBytes)
            return fail(NSOSX_ERR_INVALID, "edge_pack: integrity trailer missing or corrupt");
        char hex[65];
        sha256().hex(data, pbytes, hex);
        if (std::memcmp(hex, data + size - 64, 64) != 0)
            return fail(NSOSX_ERR_INVALID, "edge_pack: SHA-256 integrity mismatch");
        payload = pbytes;
        rd.size = payload;
    }
    const uint32_t count = rd.pod<uint32_t>();
    if (!rd.ok) return fail(NSOSX_ERR_INVALID, "edge_pack: truncated layer count");
    if ((int64_t)count > (int64_t)max_layers) {
        *num_layers = static_cast<int>(count);
        return fail(NSOSX_ERR_OVERFLOW, "edge_pack: more layers than descriptors");
    }
    for (uint32_t i = 0; i < count; ++i) {
        nsosx_edge_layer L{};
        const uint8_t sensitive = rd.pod<uint8_t>();
        L.in_features = rd.pod<int32_t>();
        L.out_features = rd.pod<int32_t>();
        const uint8_t use_bias = rd.pod<uint8_t>();
        L.weight_scale = rd.pod<float>();
        if (!rd.ok) return fail(NSOSX_ERR_INVALID, "edge_pack: truncated layer header");
        if (sensitive > 1) return fail(NSOSX_ERR_INVALID, "edge_pack: invalid sensitivity flag");
        if (use_bias > 1) return fail(NSOSX_ERR_INVALID, "edge_pack: invalid bias flag");
        if (L.in_features <= 0 || L.out_features <= 0)
            return fail(NSOSX_ERR_INVALID, "edge_pack: non-positive linear dimensions");
        if (!std::isfinite(L.weight_scale) || L.weight_scale <= 0.0f)
            return fail(NSOSX_ERR_INVALID, "edge_pack: invalid weight scale");
        L.sensitive = sensitive;
        L.use_bias = use_bias;
        const uint64_t n_in = (uint64_t)L.in_features, n_out = (uint64_t)L.out_features;
        const uint64_t weights = n_in * n_out;
        L.packed_words = (weights + 15) / 16;
        bool c1, c2, c3, c4, c5, c6 = true;
        L.packed_offset = rd.vec(L.packed_words, 4, c1);
        L.magnitude_offset = rd.vec(n_out, 4, c2);
        L.bias_offset = rd.vec(use_bias ? n_out : 0, 4, c3);
        L.alpha_offset = rd.vec(n_in, 4, c4);
        L.beta_offset = rd.vec(n_in, 4, c5);
        if (sensitive) L.sensitive_offset = rd.vec(weights, 4, c6);
        if (!(c1 && c2 && c3 && c4 && c5 && c6) || !rd.ok)
            return fail(NSOSX_ERR_INVALID,
                        "edge_pack: vector length does not match the layer metadata");
        if (!all_finite(data, L.magnitude_offset, n_out) ||
            !all_finite(data, L.bias_offset, use_bias ? n_out : 0) ||
            !all_finite(data, L.alpha_offset, n_in) || !all_finite(data, L.beta_offset, n_in) ||
            (sensitive && !all_finite(data, L.sensitive_offset, weights)))
            return fail(NSOSX_ERR_INVALID, "edge_pack: non-finite values");
        for (uint64_t w = 0; w < L.packed_words; ++w) {
            uint32_t word;
            std::memcpy(&word, data + L.packed_offset + 4 * w, 4);
            uint32_t both = word & (word >> 1) & 0x55555555u;
            const uint64_t valid = weights - w * 16;
            if (valid < 16) both &= (1u << (2 * valid)) - 1u;
            if (both) return fail(NSOSX_ERR_RESERVED, "edge_pack: reserved ternary weight code");
        }
        layers[i] = L;
    }
    if (rd.pos != payload)
        return fail(NSOSX_ERR_INVALID, version == 3
                                           ? "edge_pack: payload length does not match its trailer"
                                           : "edge_pack: trailing bytes after the last layer");
    *num_layers = static_cast<int>(count);
    return NSOSX_OK;
}
