// linear_common.h -- parameters and helpers shared by the perturbed-forward kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hses.h"
#include "bm_exact.h"
#include "mfma.h"
#include "spike_fmt.h"

namespace hses {

struct DeviceState;

__host__ __device__ constexpr size_t align16(size_t x) { return (x + 15) & ~(size_t)15; }

template <int MATH>
struct MathT;
template <>
struct MathT<HSES_MATH_F32> {
    using T = float;
    static constexpr int PAD = 4;
    __device__ static T zero() { return 0.0f; }
    __device__ static T one() { return 1.0f; }
    __device__ static T cvt(float v) { return v; }
};
template <>
struct MathT<HSES_MATH_BF16> {
    using T = uint16_t;
    static constexpr int PAD = 8;
    __device__ static T zero() { return 0; }
    __device__ static T one() { return 0x3f80; }
    __device__ static T cvt(float v) { return f2bf(v); }
};

// Everything a perturbed-forward launch needs (passed by value).
struct LinParams {
    const void* x;
    int32_t x_fmt;
    int64_t x_stride, x_plane;
    int32_t n_time, rpm;
    const float* W;
    int32_t a, b;
    uint64_t key;
    int32_t r;
    float bs;
    int32_t epoch, nreuse, tid_lo, n;
    float* y;
    int64_t y_stride, y_plane;
    int32_t math;
    // 0: do_mm, y = x W^T + (x B) A^T with W (a, b), stream rows B then A.
    // 1: do_Tmm, y = x W + (x A) B^T for a parameter W of shape (b, a) (x has
    //    b columns, y has a): the first b stream rows (its B) are the output
    //    side operand, the next a rows (its A, scaled) the input side.
    int32_t tmm;
    int32_t R;      // rows per member = n_time * rpm
    int64_t total;  // n * R
    // kernel-specific tiling
    int32_t nm_max, ne_real, ne, rc, bpitch;
    const BmTables* tables;
    const uint32_t* log_exc;
    const uint32_t* cos_exc;
    const uint64_t* jump;
    float* rec;  // factor record (pair kernels, do_mm), or NULL
    // member weights (launch_linear_mw): member tid_lo + m's at wm + m * wm_stride
    const uint16_t* wm;
    int64_t wm_stride;
};

// Physical offset (in units) of member-major logical row L: member m = L / R,
// time t and slot s inside the member; element (t, m*rpm + s).
__device__ __forceinline__ int64_t phys_row(const LinParams& P, int64_t L, int64_t stride,
                                            int64_t plane) {
    const int64_t m = L / P.R;
    const int32_t rem = (int32_t)(L - m * P.R);
    const int32_t t = rem / P.rpm;
    const int32_t s = rem - t * P.rpm;
    return t * plane + (m * P.rpm + s) * stride;
}

// Eight consecutive activations x[row][k0..k0+8) converted to the MFMA type.
// k0 is a multiple of 8; columns >= b read as zero.
template <int MATH, int XFMT>
__device__ __forceinline__ void load_x_seg(const void* x, int64_t off, bool valid, int32_t k0,
                                           int32_t b, typename MathT<MATH>::T out[8]) {
    using M = MathT<MATH>;
    if constexpr (XFMT == HSES_FMT_BITS) {
        uint32_t byte = 0;
        if (valid && k0 < b) {
            const uint64_t w = static_cast<const uint64_t*>(x)[off + (k0 >> 6)];
            byte = (uint32_t)(w >> (k0 & 63)) & 0xffu;
            if (b - k0 < 8) byte &= (1u << (b - k0)) - 1u;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) out[i] = ((byte >> i) & 1u) ? M::one() : M::zero();
    } else if constexpr (XFMT == HSES_FMT_BF16) {
        const uint16_t* p = static_cast<const uint16_t*>(x) + off;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint16_t h = (valid && k0 + i < b) ? p[k0 + i] : (uint16_t)0;
            if constexpr (MATH == HSES_MATH_BF16)
                out[i] = h;
            else
                out[i] = bf2f(h);
        }
    } else {
        const float* p = static_cast<const float*>(x) + off;
#pragma unroll
        for (int i = 0; i < 8; ++i) out[i] = M::cvt((valid && k0 + i < b) ? p[k0 + i] : 0.0f);
    }
}

// Eight bits of x (bit e = column k0 + e) as an MFMA operand of 0.0 / 1.0 bf16.
// Dword q holds elements 2q (low half) and 2q+1 (high half):
// y = byte | byte << 15 puts bit 2q at 2q and bit 2q+1 at 16 + 2q, and the
// multiply by 0x3F80 >> 2q moves both to their half-word as bf16 1.0.
__device__ __forceinline__ u16x8 expand_bits(uint32_t byte) {
    const uint32_t y = byte | (byte << 15);
    uint32_t d[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) d[q] = __umul24(y & (0x10001u << (2 * q)), 0x3F80u >> (2 * q));
    u16x8 v;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        v[2 * q] = (uint16_t)d[q];
        v[2 * q + 1] = (uint16_t)(d[q] >> 16);
    }
    return v;
}

// The same as fp16 1.0 / 0.0 (0x3C00 has its low ten bits clear, so the
// multiplies by 0x3C00 >> 2q stay exact).
__device__ __forceinline__ u16x8 expand_bits_f16(uint32_t byte) {
    const uint32_t y = byte | (byte << 15);
    uint32_t d[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) d[q] = __umul24(y & (0x10001u << (2 * q)), 0x3C00u >> (2 * q));
    u16x8 v;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        v[2 * q] = (uint16_t)d[q];
        v[2 * q + 1] = (uint16_t)(d[q] >> 16);
    }
    return v;
}

// Fused LIF output of the large-rank kernel (see hses_perturbed_linear_lif).
struct LifOut {
    void* spk;  // bit-packed spikes (T, M, words) or NULL
    int64_t spk_stride, spk_plane;
    float* rate;  // (M, a) spike rates or NULL
    int64_t rate_stride;
    float leak, v_th;
    // spike-count bit planes in place of the rates (k_pair_bits only), or NULL
    void* cpl;
    int64_t cpl_stride;
};

int launch_linear_small(LinParams& P, DeviceState* st, hipStream_t s);
// fp32 math, do_mm, rank <= 16: the members' A_m / B_m rows into the workspace,
// then an fp32 MFMA GEMM with x B_m and (x B_m) A_m^T fused (linear_f32.hip).
int launch_linear_f32(LinParams& P, DeviceState* st, hipStream_t s, void* work, size_t work_bytes);
// Every member's (a + b) x r factor rows into F (n (a + b) r floats), the
// scaled role's rows (do_mm: A; do_Tmm: the input side) times sign * sigma / sqrt(r).
int launch_factors(LinParams& P, DeviceState* st, hipStream_t s, float* F);
// bf16 math, outputs >= 256 wide, rank <= 4: the bf16 MFMA GEMM with x B_m
// fused (linear_bf16.hip); its workspace, 0 when it does not apply.
int launch_linear_bf16(LinParams& P, DeviceState* st, hipStream_t s, void* work, size_t work_bytes,
                       int32_t act, int32_t y_fmt);
size_t linear_bf16_workspace(int32_t a, int32_t b, int32_t r, int32_t n, int32_t rows_per_member,
                             int32_t n_time, int32_t math);
size_t linear_f32_workspace(int32_t a, int32_t b, int32_t r, int32_t n, int32_t rows_per_member,
                            int32_t n_time, int32_t math);
// The pair kernels (rank a multiple of 16 <= 128, output width <= 128, bf16).
// With bimg the factors were drawn ahead by launch_pair_gen: A is read from
// P.rec, B from bimg, and the kernels draw nothing.
int launch_linear_pair(LinParams& P, DeviceState* st, hipStream_t s, void* work, size_t work_bytes,
                       const LifOut* lif = nullptr, const uint16_t* bimg = nullptr);
size_t linear_pair_workspace(const DeviceState* st, int32_t a, int32_t b, int32_t r, int32_t n);
// Every pair's factors of members [tid_lo, tid_lo + n) into the record P.rec
// and the bf16 operand image bimg (pair_image_bytes bytes), or with split
// the split operand image (pair_image_x_bytes bytes).
int launch_pair_gen(LinParams& P, DeviceState* st, hipStream_t s, uint16_t* bimg,
                    bool split = false);
size_t pair_image_bytes(int32_t a, int32_t b, int32_t r, int32_t tid_lo, int32_t n);
// The split (HSES_MATH_F32X) operand image of members [tid_lo, tid_lo + n)
// from their factor record rec (do_mm, scale bs on the output side), and its
// size.  launch_linear_pair with P.math = HSES_MATH_F32X takes it as bimg.
int launch_pair_image_x(const float* rec, int32_t a, int32_t b, int32_t r, float bs, int32_t tid_lo,
                        int32_t n, uint16_t* img, hipStream_t s);
size_t pair_image_x_bytes(int32_t a, int32_t b, int32_t r, int32_t tid_lo, int32_t n);
// Member weights (linear_mw.hip): W_m = W + sign_m bs A_m B_m^T of members
// [tid_lo, tid_lo + n) from their factor record, bf16 (a, kp) per member or,
// split, the fp16 high and low parts of 1024 W_m; and the forward on them
// (P.wm, P.wm_stride; bit-packed x, rows per member a multiple of 256).
size_t member_weights_bytes(int32_t a, int32_t b, int32_t n, bool split);
int launch_member_weights(const float* W, const float* rec, int32_t a, int32_t b, int32_t r,
                          float bs, int32_t tid_lo, int32_t n, bool split, uint16_t* wm,
                          hipStream_t s);
int launch_linear_mw(LinParams& P, DeviceState* st, hipStream_t s, const LifOut* lif);
// The readout on count planes with member weights formed in LDS
// (k_readout_counts): a <= 32, b <= 128, 2 rows per member <= 256, T <= 16.
size_t readout_counts_lds(int32_t a, int32_t b, int32_t r);
int launch_readout_counts(const uint64_t* cpl, int64_t cstride, int32_t T, const float* W,
                          int32_t a, int32_t b, int32_t r, float bs, int32_t tid_lo, int32_t n,
                          int32_t rpm, const float* rec, float* y, int64_t ystride,
                          hipStream_t s);
// The wide small-rank kernel: 0 when it does not apply to the shape, else its
// workspace (W as bf16, (a, kp)).
size_t linear_wide_workspace(int32_t a, int32_t b, int32_t r, int32_t n, int32_t rows_per_member,
                             int32_t n_time, int32_t math);
int launch_linear_wide(LinParams& P, DeviceState* st, hipStream_t s, void* work, size_t work_bytes,
                       int32_t act, int32_t y_fmt = HSES_FMT_F32);
// W (a, b) fp32 -> (a, kp) bf16, zero columns [b, kp); tmm: W is stored (b, a).
void launch_w_to_bf16(const float* W, int32_t a, int32_t b, int32_t kp, int32_t tmm, uint16_t* out,
                      hipStream_t s);

// Elementwise activation fused into a forward epilogue (hses_act).
enum { ACT_NONE = HSES_ACT_NONE, ACT_TANH = HSES_ACT_TANH, ACT_SIGMOID = HSES_ACT_SIGMOID,
       ACT_RELU_SQ = HSES_ACT_RELU_SQ };

// Rows of a tile: row L0 + i (i within the tile) is member m_first + dm of the tile
// with dm, its time plane and slot from 32-bit divisions of rem0 + i (the
// 64-bit division by R happens once per workgroup).
struct TileRows {
    int32_t m_first, rem0;
    __device__ __forceinline__ TileRows(const LinParams& P, int64_t L0) {
        m_first = (int32_t)(L0 / P.R);
        rem0 = (int32_t)(L0 - (int64_t)m_first * P.R);
    }
    __device__ __forceinline__ int32_t member(const LinParams& P, int32_t i) const {
        return (rem0 + i) / P.R;
    }
    __device__ __forceinline__ int64_t offset(const LinParams& P, int32_t i, int64_t stride,
                                              int64_t plane) const {
        const int32_t rr = rem0 + i, dm = rr / P.R, rem = rr - dm * P.R;
        const int32_t t = rem / P.rpm, s = rem - t * P.rpm;
        return t * plane + ((int64_t)(m_first + dm) * P.rpm + s) * stride;
    }
};

}  // namespace hses
