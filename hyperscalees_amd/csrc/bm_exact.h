// bm_exact.h -- the noiser's Box-Muller normal, reproduced bit for bit on the GPU.
//
// The reference draws each factor entry as (noiser.rs:448-477)
//     k1, k2 = 24-bit unit indices of two xorshift64 steps
//     u1 = max(k1 * 2^-24, 1e-9f);  u2 = k2 * 2^-24
//     n  = sqrtf(-2 * logf(u1)) * cosf(TAU * u2)          (f32 throughout)
// with logf/cosf from glibc.  glibc's results are not correctly rounded for
// about 1% of the 2^24 possible inputs, so the device evaluates log and cos in
// f64 with the table-driven routines below (only IEEE +, *, fma and
// conversions, so the host compiler and hipcc produce identical bits), rounds
// to f32, and corrects the inputs where glibc differs with a per-input
// exception bitmap.  A bitmap word is read only when the f64 result lies close
// to an f32 rounding midpoint ("danger" test): every glibc exception lies in
// that zone, and outside it the correctly rounded value is glibc's value.  The
// host builds the tables and bitmaps (bm_tables.cpp) with this same code, so
// the danger test agrees bit for bit on host and device.
//
// This file is included by host C++ (g++, -ffp-contract=off) and by HIP device
// code (hipcc, -ffp-contract=off).  Nothing here may depend on a libm routine.
#pragma once
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define HSES_HD __host__ __device__ __forceinline__
#else
#include <math.h>
#define HSES_HD inline
#endif

namespace hses {

// Table sizes.
constexpr int kLogTab = 128;          // subintervals of the reduced argument z in [0.75, 1.5)
constexpr int kCosTab = 64;           // angle grid j * 2pi / 64, j = 0..64
constexpr int kBucketShift = 17;      // danger-threshold buckets: k >> kBucketShift
constexpr int kBuckets = 1 << (24 - kBucketShift);
constexpr uint32_t kUnitCount = 1u << 24;
constexpr uint32_t kBitmapWords = kUnitCount / 32;
// Bitmaps are stored with 64 zero words appended: lanes without a danger test
// read word kBitmapWords, so their loaded bits need no masking.
constexpr uint32_t kBitmapAlloc = kBitmapWords + 64;

// Danger window of one bucket: rem29(y) in [2^28 - t, 2^28 + t) for a
// half-width t (units of 2^-29 f32 ulp), stored as lo = 2^28 - t and w = 2t so
// the test is one subtraction and one unsigned compare.
struct DangerWin {
    uint32_t lo, w;
};

// Small per-function tables (copied into LDS by kernels).
struct BmTables {
    double log_invc[kLogTab];
    double log_logc[kLogTab];
    double cos_c[kCosTab + 1];
    double cos_s[kCosTab + 1];
    double cos_thi[kCosTab + 1];
    double cos_tlo[kCosTab + 1];
    DangerWin log_dw[kBuckets];
    DangerWin cos_dw[kBuckets];
};

HSES_HD uint32_t f2u(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __float_as_uint(f);
#else
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
#endif
}
HSES_HD float u2f(uint32_t u) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __uint_as_float(u);
#else
    float f;
    memcpy(&f, &u, 4);
    return f;
#endif
}

HSES_HD double hfma(double a, double b, double c) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_fma(a, b, c);
#else
    return fma(a, b, c);
#endif
}

// fma with a compile-time constant addend.  On the device the constant sits in
// a scalar register pair as the third operand of v_fma_f64 (the two-address
// v_fmac form would copy it into the destination first).
HSES_HD double hfma_k(double a, double b, double c) {
#if defined(__HIP_DEVICE_COMPILE__)
    double d;
    asm("v_fma_f64 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "s"(c));
    return d;
#else
    return fma(a, b, c);
#endif
}

HSES_HD float hfmax(float a, float b) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_fmaxf(a, b);
#else
    return fmaxf(a, b);
#endif
}

// Constants shared by host and device.
constexpr double kLn2Hi = 6.93147180369123816490e-01;  // 0x3FE62E42FEE00000, 32 significant bits
constexpr double kLn2Lo = 1.90821492927058770002e-10;  // 0x3DEA39EF35793C76
constexpr float kTauF = 6.28318530717958647692f;       // std::f32::consts::TAU

// Polynomial coefficients (Taylor, rounded to double).  The degrees only set
// how often the f64 value lands near an f32 rounding midpoint: every input
// where glibc differs from RN32 of these routines is an exception in the
// bitmaps (checked over all 2^24 inputs when the tables are built), so
// correctness does not depend on them.  Truncation errors: log1p to r^3,
// |r| <= 2^-8: < 2^-34 absolute, about 2^-10 f32 ulp where |log x| >= 2^-8
// (relative on the two c = 1 subintervals); cos to t^4 and sin to t^5,
// |t| <= pi/64: < 2^-35 absolute against |cos| >= 2^-4.4 off the quadrant
// points, where c_j = 0 and only the (relative) sin series counts.  Both stay
// far inside glibc's own error (danger windows of ~0.3 ulp), so the
// exception bitmaps and danger rates barely change with the degree.
constexpr double kL2 = -0.5, kL3 = 1.0 / 3.0;
constexpr double kC2 = -0.5, kC4 = 1.0 / 24.0;
constexpr double kS3 = -1.0 / 6.0, kS5 = 1.0 / 120.0;

// The f32 argument of logf for unit index k1: max(k1 * 2^-24, 1e-9f)
// (noiser.rs:474); only k1 == 0 is clamped, every other k1 * 2^-24 >= 2^-24.
HSES_HD float log_arg(uint32_t k1) { return hfmax((float)(int32_t)k1 * 0x1p-24f, 1e-9f); }

// The f32 angle TAU * (k2 * 2^-24) of noiser.rs:475-476, as one multiply:
// k2 * 2^-24 is exact (k2 < 2^24) and so is TAU * 2^-24, so both forms round
// the same real product once.
constexpr float kTauLsb = kTauF * 0x1p-24f;
HSES_HD float cos_arg(uint32_t k2) { return (float)(int32_t)k2 * kTauLsb; }

// f64 evaluation of log(x) for x = log_arg(k1) (x in [1e-9, 1); any positive
// normal f32 works).
// x = 2^E * z with z in [0.75, 1.5); log x = E ln2 + logc + log1p(z*invc - 1).
HSES_HD double log_f64(float x, const double* invc_tab, const double* logc_tab) {
    const uint32_t ix = f2u(x);
    const uint32_t tmp = ix - 0x3f400000u;  // 0.75f
    const int32_t E = (int32_t)tmp >> 23;
    const uint32_t idx = (tmp >> 16) & (kLogTab - 1);
    const uint32_t iz = ix - ((uint32_t)E << 23);
    const double z = (double)u2f(iz);
    const double r = hfma(z, invc_tab[idx], -1.0);
    const double p = hfma_k(r, kL3, kL2);
    const double r2 = r * r;
    const double lp = hfma(r2, p, r);
    const double Ed = (double)E;
    const double hi = hfma(Ed, kLn2Hi, logc_tab[idx]);
    const double lo = hfma(Ed, kLn2Lo, lp);
    return hi + lo;
}

// f64 evaluation of cos(th) for th = cos_arg(k2) = TAU * k2 * 2^-24 (th in
// [0, 2pi)).  th = theta_j + t with theta_j = j * 2pi/64 and j = round(k2 /
// 2^18), the grid point of the unrounded angle 2pi * k2 / 2^24 (th differs
// from it by < 3e-8 relative, so |t| <= pi/64 * (1 + 4e-6));
// cos th = c_j cos t - s_j sin t.
HSES_HD double cos_f64(float th, uint32_t k2, const double* c_tab, const double* s_tab,
                       const double* thi_tab, const double* tlo_tab) {
    const double x = (double)th;
    const uint32_t j = (k2 + (1u << 17)) >> 18;
    const double t = (x - thi_tab[j]) - tlo_tab[j];
    const double t2 = t * t;
    const double pc = hfma_k(t2, kC4, kC2);
    const double ct = hfma(t2, pc, 1.0);
    const double ps = hfma_k(t2, kS5, kS3);
    const double st = hfma(t * t2, ps, t);
    const double sj = s_tab[j] * st;
    return hfma(c_tab[j], ct, -sj);
}

HSES_HD uint64_t d2u(double d) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __double_as_longlong(d);
#else
    uint64_t u;
    memcpy(&u, &d, 8);
    return u;
#endif
}

// Rounding y (a normal-range f64) to f32 keeps the top 23 of its 52 mantissa
// bits; the low 29 bits R (the low word's bits 0..28) decide the rounding,
// with the midpoint at R = 2^28.  |R - 2^28| is the distance to the nearest
// rounding midpoint in units of 2^-29 f32 ulp.
HSES_HD uint32_t rem29(double y) { return (uint32_t)d2u(y) & 0x1FFFFFFFu; }

// Inside the bucket's window around the midpoint (one unsigned compare).
HSES_HD bool in_danger_r(uint32_t R, DangerWin d) { return R - d.lo < d.w; }
HSES_HD bool in_danger(double y, DangerWin d) { return in_danger_r(rem29(y), d); }

// The other f32 candidate for y: the neighbour of f = RN32(y) across the
// nearest rounding midpoint (the only other value glibc's logf/cosf return).
// R = rem29(y) > 2^28 means y was rounded up in magnitude (|f| > |y|), so the
// other candidate is one step toward zero; otherwise one step away.  (An
// exact tie, R = 2^28, would be misjudged when it rounds down; the table
// builder checks this rule against glibc for every exception.)
HSES_HD float other_candidate(float f, uint32_t R) {
    return u2f(R > 0x10000000u ? f2u(f) - 1u : f2u(f) + 1u);
}

// ---------------------------------------------------------------------------
// Integer stream: noise_seed, xorshift64 and GF(2) jump-ahead.
// ---------------------------------------------------------------------------

// noiser.rs:495-506; i32 widens with sign extension as Rust's `as u64` does.
HSES_HD uint64_t noise_seed(uint64_t key, int32_t true_epoch, int32_t true_thread) {
    uint64_t h = key ^ 0x9E3779B97F4A7C15ull;
    h *= 0xBF58476D1CE4E5B9ull;
    h ^= (uint64_t)(int64_t)true_epoch * 0x94D049BB133111EBull;
    h = ((h << 17) | (h >> 47)) ^ (uint64_t)(int64_t)true_thread;
    h ^= h >> 33;
    h *= 0xBF58476D1CE4E5B9ull;
    h ^= h >> 29;
    h *= 0x94D049BB133111EBull;
    h ^= h >> 32;
    return h;
}

// noiser.rs:453-460
HSES_HD uint64_t xs64(uint64_t x) {
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    return x;
}

// Entries of a GF(2) matrix in nibble form (16 nibble positions x 16 values).
constexpr int kJumpNib = 256;

// y = J x over GF(2), J given by its 64 columns (column i = J e_i).
HSES_HD uint64_t gf2_apply(const uint64_t* cols, uint64_t x) {
    uint64_t y = 0;
#if defined(__HIP_DEVICE_COMPILE__)
#pragma unroll 4
#endif
    for (int i = 0; i < 64; ++i) y ^= (0ull - ((x >> i) & 1ull)) & cols[i];
    return y;
}

// eggroll.rs:60-65
HSES_HD void epoch_thread_sign(int32_t epoch, int32_t tid, int32_t noise_reuse, int32_t* te,
                               int32_t* tt, float* sign) {
    *te = noise_reuse == 0 ? 0 : epoch / noise_reuse;
    *tt = tid / 2;
    *sign = (tid % 2 == 0) ? 1.0f : -1.0f;
}

}  // namespace hses
