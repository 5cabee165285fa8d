// spike_fmt.h -- storage of 0/1 activations in the formats of hses_fmt.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hses.h"

namespace hses {

// Rows of `units` elements at row * stride + t * plane (row < M, t < n_time)
// do not overlap: time-major (planes of M rows, plane >= M * stride) or
// time-inner (each row's n_time entries adjacent, stride >= n_time * plane).
inline bool rows_layout_ok(int64_t units, int64_t M, int32_t n_time, int64_t stride,
                           int64_t plane) {
    if (n_time <= 1) return stride >= units;
    return (stride >= units && plane >= M * stride) || (plane >= units && stride >= n_time * plane);
}

// Row length, in storage units, of a row of `width` spikes.
inline int64_t fmt_row_units(int32_t fmt, int64_t width) {
    return fmt == HSES_FMT_BITS ? (width + 63) / 64 : width;
}
inline int64_t fmt_unit_bytes(int32_t fmt) {
    switch (fmt) {
        case HSES_FMT_F32: return 4;
        case HSES_FMT_BF16: return 2;
        case HSES_FMT_U8: return 1;
        default: return 8;
    }
}

// Store one spike.  `base` is the offset (in units) of the row; every lane of
// the wave must call this (BITS uses a wave-wide ballot; lane 0 stores the word).
template <int FMT>
__device__ __forceinline__ void store_spike(void* out, int64_t base, int32_t word, int32_t col,
                                            bool valid, bool spike) {
    if constexpr (FMT == HSES_FMT_BITS) {
        const uint64_t bits = __ballot(spike);
        if ((threadIdx.x & 63) == 0) static_cast<uint64_t*>(out)[base + word] = bits;
    } else if constexpr (FMT == HSES_FMT_F32) {
        if (valid) static_cast<float*>(out)[base + col] = spike ? 1.0f : 0.0f;
    } else if constexpr (FMT == HSES_FMT_BF16) {
        if (valid) static_cast<uint16_t*>(out)[base + col] = spike ? (uint16_t)0x3f80 : (uint16_t)0;
    } else {
        if (valid) static_cast<uint8_t*>(out)[base + col] = spike ? 1 : 0;
    }
}

}  // namespace hses
