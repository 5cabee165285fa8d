// spiking.hip -- Poisson rate encoding and the LIF scan, HBM-streaming kernels.
//
// Both kernels map one wavefront to 64 consecutive columns of one row: loads
// and stores of a time plane are contiguous across the wave, and the packed
// spike format is one __ballot per (time step, row, 64 columns) written by a
// single lane.
#include "runtime.h"
#include "spike_fmt.h"

namespace hses {

// Largest m in [0, 2^23] such that m == 0 or RN32(m / 8388609) < p.  The
// reference compares u = ((v >> 9) + 1) / 8388609 (f32 division) with p
// (poisson_encode_fused_oxide.rs:44-52); since RN32(m / D) is non-decreasing
// in m, `u < p` is exactly `(v >> 9) + 1 <= K(p)`.  floor(p*D) is exact in
// f64 and the rounding of m/D moves the crossing by less than one step, so
// only three candidates need the (correctly rounded) f32 division.
__device__ __forceinline__ uint32_t poisson_threshold(float p) {
    if (!(p > 0.0f)) return 0u;  // p <= 0 or NaN: never fires
    const double pd = (double)p * 8388609.0;
    const double fl = __builtin_floor(pd);
    const uint32_t m0 = fl >= 8388608.0 ? 8388608u : (uint32_t)fl;
    auto lt = [p](uint32_t m) { return (float)m / 8388609.0f < p; };
    if (m0 < 8388608u && lt(m0 + 1u)) return m0 + 1u;
    if (m0 >= 1u && lt(m0)) return m0;
    return m0 >= 1u ? m0 - 1u : 0u;
}

template <int FMT>
__global__ __launch_bounds__(256) void k_poisson(const float* __restrict__ p, int64_t p_rows,
                                                 const int32_t* __restrict__ prow, int64_t rows,
                                                 int32_t in_dim, int64_t p_stride, int32_t T,
                                                 uint32_t mix, void* __restrict__ out,
                                                 int64_t out_stride) {
    const int32_t words = (in_dim + 63) >> 6;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int32_t lane = threadIdx.x & 63;
    if (wave >= rows * words) return;  // whole wave exits together
    const int64_t row = wave / words;
    const int32_t word = (int32_t)(wave % words);
    const int32_t col = word * 64 + lane;
    const bool valid = col < in_dim;
    uint32_t K = 0, x = 0;
    if (valid) {
        const int64_t src = prow ? (int64_t)prow[row] : row;
        K = (src >= 0 && src < p_rows) ? poisson_threshold(p[src * p_stride + col]) : 0u;
        const uint32_t idx = (uint32_t)(row * in_dim + col);
        x = 1000000007u * idx + mix + 0x9E3779B9u;
    }
    const int64_t plane = rows * out_stride;
    for (int32_t t = 0; t < T; ++t) {
        x ^= x << 13;
        x ^= x >> 17;
        x ^= x << 5;
        const bool spike = valid && ((x >> 9) + 1u) <= K;
        store_spike<FMT>(out, t * plane + row * out_stride, word, col, valid, spike);
    }
}

template <int FMT>
__global__ __launch_bounds__(256) void k_lif(const float* __restrict__ cur,
                                             const float* __restrict__ v0, int32_t T, int64_t rows,
                                             int32_t h, int64_t cur_stride, float leak, float v_th,
                                             void* __restrict__ spk, int64_t spk_stride,
                                             float* __restrict__ v_out) {
    const int32_t words = (h + 63) >> 6;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int32_t lane = threadIdx.x & 63;
    if (wave >= rows * words) return;
    const int64_t row = wave / words;
    const int32_t word = (int32_t)(wave % words);
    const int32_t col = word * 64 + lane;
    const bool valid = col < h;
    float v = (valid && v0) ? v0[row * h + col] : 0.0f;
    const int64_t cplane = rows * cur_stride, splane = rows * spk_stride;
    const float* cp = cur + row * cur_stride + col;
    for (int32_t t = 0; t < T; ++t) {
        const float c = valid ? cp[t * cplane] : 0.0f;
        // snn.rs:61-63: charged = v + ((-v) + c) * leak; each op rounds.
        const float charged = __fadd_rn(v, __fmul_rn(__fadd_rn(-v, c), leak));
        const bool spike = charged >= v_th;
        v = __fmul_rn(charged, __fadd_rn(spike ? -1.0f : -0.0f, 1.0f));
        store_spike<FMT>(spk, t * splane + row * spk_stride, word, col, valid, spike);
    }
    if (valid && v_out) v_out[row * h + col] = v;
}

// snn.rs:274: spikes.mean_dim(0) -- the count of spikes over T divided by T.
template <int FMT>
__global__ __launch_bounds__(256) void k_spike_rate(const void* __restrict__ spk, int64_t stride,
                                                    int32_t T, int64_t rows, int32_t h,
                                                    float* __restrict__ rate) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= rows * h) return;
    const int64_t row = e / h;
    const int32_t c = (int32_t)(e % h);
    const int64_t plane = rows * stride;
    int32_t cnt = 0;
    for (int32_t t = 0; t < T; ++t) {
        const int64_t base = t * plane + row * stride;
        if constexpr (FMT == HSES_FMT_BITS)
            cnt += (int32_t)((static_cast<const uint64_t*>(spk)[base + (c >> 6)] >> (c & 63)) & 1ull);
        else if constexpr (FMT == HSES_FMT_F32)
            cnt += static_cast<const float*>(spk)[base + c] != 0.0f;
        else if constexpr (FMT == HSES_FMT_BF16)
            cnt += static_cast<const uint16_t*>(spk)[base + c] != 0;
        else
            cnt += static_cast<const uint8_t*>(spk)[base + c] != 0;
    }
    rate[e] = __fdiv_rn((float)cnt, (float)T);
}

}  // namespace hses

using namespace hses;

extern "C" int hses_spike_rate(const void* d_spikes, int32_t fmt, int64_t spk_stride, int32_t T,
                               int64_t rows, int32_t h, float* d_rate, void* stream) {
    HSES_REQUIRE(fmt >= HSES_FMT_F32 && fmt <= HSES_FMT_BITS, "unknown spike format");
    HSES_REQUIRE(rows >= 0 && h >= 0 && T >= 1, "bad sizes");
    if (rows == 0 || h == 0) return HSES_OK;
    HSES_REQUIRE(d_spikes && d_rate, "NULL pointer");
    HSES_REQUIRE(spk_stride >= fmt_row_units(fmt, h), "spk_stride too small for format");
    const int64_t blocks = (rows * h + 255) / 256;
    HSES_REQUIRE(blocks < (1ll << 31), "grid too large");
    hipStream_t s = (hipStream_t)stream;
    switch (fmt) {
        case HSES_FMT_F32:
            hipLaunchKernelGGL(k_spike_rate<HSES_FMT_F32>, dim3(blocks), dim3(256), 0, s, d_spikes, spk_stride, T, rows, h, d_rate);
            break;
        case HSES_FMT_BF16:
            hipLaunchKernelGGL(k_spike_rate<HSES_FMT_BF16>, dim3(blocks), dim3(256), 0, s, d_spikes, spk_stride, T, rows, h, d_rate);
            break;
        case HSES_FMT_U8:
            hipLaunchKernelGGL(k_spike_rate<HSES_FMT_U8>, dim3(blocks), dim3(256), 0, s, d_spikes, spk_stride, T, rows, h, d_rate);
            break;
        default:
            hipLaunchKernelGGL(k_spike_rate<HSES_FMT_BITS>, dim3(blocks), dim3(256), 0, s, d_spikes, spk_stride, T, rows, h, d_rate);
            break;
    }
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

static int64_t wave_blocks(int64_t rows, int32_t width) {
    const int64_t waves = rows * ((width + 63) / 64);
    return (waves + 3) / 4;  // 4 waves per 256-thread block
}

extern "C" int hses_poisson_encode(const float* d_p, int64_t p_rows, const int32_t* d_rows, int64_t rows,
                                   int32_t in_dim, int64_t p_stride, int32_t T, uint32_t s0,
                                   uint32_t s1, uint32_t s2, uint32_t s3, void* d_out, int32_t fmt,
                                   int64_t out_stride, void* stream) {
    HSES_REQUIRE(rows >= 0 && in_dim >= 0 && T >= 0, "negative size");
    HSES_REQUIRE(fmt >= HSES_FMT_F32 && fmt <= HSES_FMT_BITS, "unknown spike format");
    if (rows == 0 || in_dim == 0 || T == 0) return HSES_OK;
    HSES_REQUIRE(d_p && d_out, "NULL pointer");
    HSES_REQUIRE(p_stride >= in_dim, "p_stride < in_dim");
    HSES_REQUIRE(d_rows || p_rows >= rows, "p_rows < rows without a row index");
    HSES_REQUIRE(out_stride >= fmt_row_units(fmt, in_dim), "out_stride too small for format");
    // The reference seeds with the flat index as u32 (poisson_encode_fused_oxide.rs:68-83).
    HSES_REQUIRE(rows * in_dim <= (int64_t)UINT32_MAX, "rows*in_dim exceeds the u32 index range");
    const int64_t blocks = wave_blocks(rows, in_dim);
    HSES_REQUIRE(blocks < (1ll << 31), "grid too large");
    const uint32_t mix = s0 ^ s1 ^ s2 ^ s3;
    hipStream_t s = (hipStream_t)stream;
    switch (fmt) {
        case HSES_FMT_F32:
            hipLaunchKernelGGL(k_poisson<HSES_FMT_F32>, dim3(blocks), dim3(256), 0, s, d_p, p_rows, d_rows,
                               rows, in_dim, p_stride, T, mix, d_out, out_stride);
            break;
        case HSES_FMT_BF16:
            hipLaunchKernelGGL(k_poisson<HSES_FMT_BF16>, dim3(blocks), dim3(256), 0, s, d_p, p_rows, d_rows,
                               rows, in_dim, p_stride, T, mix, d_out, out_stride);
            break;
        case HSES_FMT_U8:
            hipLaunchKernelGGL(k_poisson<HSES_FMT_U8>, dim3(blocks), dim3(256), 0, s, d_p, p_rows, d_rows,
                               rows, in_dim, p_stride, T, mix, d_out, out_stride);
            break;
        default:
            hipLaunchKernelGGL(k_poisson<HSES_FMT_BITS>, dim3(blocks), dim3(256), 0, s, d_p, p_rows, d_rows,
                               rows, in_dim, p_stride, T, mix, d_out, out_stride);
            break;
    }
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_lif_scan(const float* d_cur, const float* d_v0, int32_t T, int64_t rows,
                             int32_t h, int64_t cur_stride, float tau_m, float v_th,
                             void* d_spikes, int32_t fmt, int64_t spk_stride, float* d_v_out,
                             void* stream) {
    HSES_REQUIRE(rows >= 0 && h >= 0 && T >= 0, "negative size");
    HSES_REQUIRE(fmt >= HSES_FMT_F32 && fmt <= HSES_FMT_BITS, "unknown spike format");
    HSES_REQUIRE(tau_m != 0.0f, "tau_m must be non-zero");
    if (rows == 0 || h == 0) return HSES_OK;
    HSES_REQUIRE(d_cur || T == 0, "cur is NULL");
    HSES_REQUIRE(d_spikes || T == 0, "spikes is NULL");
    HSES_REQUIRE(cur_stride >= h, "cur_stride < h");
    HSES_REQUIRE(spk_stride >= fmt_row_units(fmt, h), "spk_stride too small for format");
    const int64_t blocks = wave_blocks(rows, h);
    HSES_REQUIRE(blocks < (1ll << 31), "grid too large");
    // snn.rs:59: leak_scale = dt / tau_m with dt = 1, one f32 division.
    const float leak = 1.0f / tau_m;
    hipStream_t s = (hipStream_t)stream;
    switch (fmt) {
        case HSES_FMT_F32:
            hipLaunchKernelGGL(k_lif<HSES_FMT_F32>, dim3(blocks), dim3(256), 0, s, d_cur, d_v0, T,
                               rows, h, cur_stride, leak, v_th, d_spikes, spk_stride, d_v_out);
            break;
        case HSES_FMT_BF16:
            hipLaunchKernelGGL(k_lif<HSES_FMT_BF16>, dim3(blocks), dim3(256), 0, s, d_cur, d_v0, T,
                               rows, h, cur_stride, leak, v_th, d_spikes, spk_stride, d_v_out);
            break;
        case HSES_FMT_U8:
            hipLaunchKernelGGL(k_lif<HSES_FMT_U8>, dim3(blocks), dim3(256), 0, s, d_cur, d_v0, T,
                               rows, h, cur_stride, leak, v_th, d_spikes, spk_stride, d_v_out);
            break;
        default:
            hipLaunchKernelGGL(k_lif<HSES_FMT_BITS>, dim3(blocks), dim3(256), 0, s, d_cur, d_v0, T,
                               rows, h, cur_stride, leak, v_th, d_spikes, spk_stride, d_v_out);
            break;
    }
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}
