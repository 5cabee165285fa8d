// data.cpp -- the host-side data path of the SNN ES driver: IDX/MNIST parsing
// (plain or gzip) and the driver's deterministic batch sampler.  No device code.
//
// References: read_idx_images / read_idx_labels / gunzip_if_needed
// (burn_impl/hyperscalees-envs/src/snn_mnist.rs:39-112) and shuffled_indices
// (burn_impl/hyperscalees/src/bin/accumulate_train.rs:157-174).
#include <stdint.h>
#include <string.h>
#include <zlib.h>

#include <string>
#include <vector>

#include "runtime.h"

namespace hses {

namespace {

constexpr uint32_t kIdxImages = 0x803, kIdxLabels = 0x801;  // snn_mnist.rs:17-19
constexpr uint64_t kMaxElems = 1ull << 30;                  // snn_mnist.rs:22

uint32_t be32(const uint8_t* p) {
    return (uint32_t)p[0] << 24 | (uint32_t)p[1] << 16 | (uint32_t)p[2] << 8 | (uint32_t)p[3];
}

// The buffer itself, or its gzip decompression when it starts with 1f 8b.
bool gunzip_if_needed(const uint8_t* data, size_t len, std::vector<uint8_t>* out,
                      const uint8_t** raw, size_t* raw_len, std::string* err) {
    if (len < 2 || data[0] != 0x1f || data[1] != 0x8b) {
        *raw = data;
        *raw_len = len;
        return true;
    }
    z_stream zs;
    memset(&zs, 0, sizeof(zs));
    if (inflateInit2(&zs, 16 + MAX_WBITS) != Z_OK) {
        *err = "gzip: inflateInit2 failed";
        return false;
    }
    zs.next_in = const_cast<Bytef*>(data);
    zs.avail_in = (uInt)len;  // MNIST files are far below 4 GiB
    out->resize(len * 4 + 1024);
    int rc;
    do {
        if (zs.total_out == out->size()) {
            if (out->size() > (size_t)kMaxElems + 64) {
                inflateEnd(&zs);
                *err = "gzip: decompressed size out of range";
                return false;
            }
            out->resize(out->size() * 2);
        }
        zs.next_out = out->data() + zs.total_out;
        zs.avail_out = (uInt)(out->size() - zs.total_out);
        rc = inflate(&zs, Z_NO_FLUSH);
    } while (rc == Z_OK);
    const size_t n = zs.total_out;
    inflateEnd(&zs);
    if (rc != Z_STREAM_END) {
        *err = "gzip: corrupt or truncated stream";
        return false;
    }
    out->resize(n);
    *raw = out->data();
    *raw_len = n;
    return true;
}

}  // namespace
}  // namespace hses

using namespace hses;

extern "C" int hses_read_idx_images(const uint8_t* data, size_t len, float* out, int64_t out_cap,
                                    int64_t* n_images, int64_t* pixels) {
    HSES_REQUIRE(data || len == 0, "NULL pointer");
    HSES_REQUIRE(n_images && pixels, "NULL pointer");
    std::vector<uint8_t> buf;
    const uint8_t* raw;
    size_t rl;
    std::string err;
    if (!gunzip_if_needed(data, len, &buf, &raw, &rl, &err)) return set_error(HSES_ERR_INVALID_ARG, err);
    HSES_REQUIRE(rl >= 16, "images IDX buffer too short for header");
    const uint32_t magic = be32(raw);
    if (magic != kIdxImages) return set_error(HSES_ERR_INVALID_ARG, "expected images magic 0x803");
    const uint64_t n = be32(raw + 4), rows = be32(raw + 8), cols = be32(raw + 12);
    const uint64_t per = rows * cols;  // factors below 2^32: no wrap
    HSES_REQUIRE(n <= kMaxElems && per <= kMaxElems && n * per <= kMaxElems,
                 "images payload size out of range");
    const uint64_t total = n * per;
    HSES_REQUIRE(16 + total <= rl, "images payload underflow");
    *n_images = (int64_t)n;
    *pixels = (int64_t)per;
    if (!out) return HSES_OK;
    HSES_REQUIRE(out_cap >= (int64_t)total, "out holds fewer than n * rows * cols floats");
    for (uint64_t i = 0; i < total; ++i) out[i] = (float)raw[16 + i] / 255.0f;
    return HSES_OK;
}

extern "C" int hses_read_idx_labels(const uint8_t* data, size_t len, uint8_t* out, int64_t out_cap,
                                    int64_t* n_labels) {
    HSES_REQUIRE(data || len == 0, "NULL pointer");
    HSES_REQUIRE(n_labels, "NULL pointer");
    std::vector<uint8_t> buf;
    const uint8_t* raw;
    size_t rl;
    std::string err;
    if (!gunzip_if_needed(data, len, &buf, &raw, &rl, &err)) return set_error(HSES_ERR_INVALID_ARG, err);
    HSES_REQUIRE(rl >= 8, "labels IDX buffer too short for header");
    if (be32(raw) != kIdxLabels) return set_error(HSES_ERR_INVALID_ARG, "expected labels magic 0x801");
    const uint64_t n = be32(raw + 4);
    HSES_REQUIRE(n <= kMaxElems && 8 + n <= rl, "labels payload underflow");
    *n_labels = (int64_t)n;
    if (!out) return HSES_OK;
    HSES_REQUIRE(out_cap >= (int64_t)n, "out holds fewer than n labels");
    memcpy(out, raw + 8, n);
    return HSES_OK;
}

extern "C" int hses_shuffled_indices(int64_t n, int64_t count, uint64_t seed, int64_t* out) {
    HSES_REQUIRE(n >= 0 && count >= 0 && count <= n, "need 0 <= count <= n");
    if (count == 0) return HSES_OK;
    HSES_REQUIRE(out, "NULL pointer");
    uint64_t state = (seed ^ 0x9E3779B97F4A7C15ull) | 1ull;
    std::vector<int64_t> idx((size_t)n);
    for (int64_t i = 0; i < n; ++i) idx[(size_t)i] = i;
    // partial Fisher-Yates over the first `count` positions; each draw is one
    // xorshift64 (13, 7, 17) step times 0x2545F4914F6CDD1D, reduced mod n - i
    for (int64_t i = 0; i < count; ++i) {
        state ^= state << 13;
        state ^= state >> 7;
        state ^= state << 17;
        const uint64_t draw = state * 0x2545F4914F6CDD1Dull;
        const int64_t j = i + (int64_t)(draw % (uint64_t)(n - i));
        const int64_t t = idx[(size_t)i];
        idx[(size_t)i] = idx[(size_t)j];
        idx[(size_t)j] = t;
    }
    memcpy(out, idx.data(), sizeof(int64_t) * (size_t)count);
    return HSES_OK;
}
