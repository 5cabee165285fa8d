// noise_dev.h -- device side of the noiser stream (see bm_exact.h).
//
// A factor stream for (layer key, epoch', pair) is the row-major sequence of
// normals of an (rows x L) matrix; normal p consumes xorshift64 states 2p+1
// and 2p+2 after s0 = noise_seed(...) | 1 (noiser.rs:437-490).  Kernels give
// each thread whole rows: the state at the start of row j is
// M^(2Lj) s0 = T1[j/16] (T0[j%16] s0), two GF(2) products with matrices from
// the per-L jump table, after which the thread steps sequentially.
#pragma once
#include <hip/hip_runtime.h>

#include "bm_exact.h"

namespace hses {

// Cooperative copy of the small tables into LDS.
__device__ __forceinline__ void load_bm_tables(BmTables* lds, const BmTables* g) {
    const uint32_t* src = reinterpret_cast<const uint32_t*>(g);
    uint32_t* dst = reinterpret_cast<uint32_t*>(lds);
    constexpr int words = sizeof(BmTables) / 4;
    for (int i = threadIdx.x; i < words; i += blockDim.x) dst[i] = src[i];
}

__device__ __forceinline__ bool bit_set(const uint32_t* bm, uint32_t k) {
    return (bm[k >> 5] >> (k & 31)) & 1u;
}

// glibc logf(max(k1 * 2^-24, 1e-9f)), bit-exact.
__device__ __forceinline__ float bm_logf(uint32_t k1, const BmTables& t, const uint32_t* exc) {
    const float x = log_arg(k1);
    const double y = log_f64(x, t.log_invc, t.log_logc);
    float g;
    bool danger;
    float f = round_with_danger(y, t.log_q[k1 >> 16], &g, &danger);
    if (danger && bit_set(exc, k1)) f = g;
    return k1 == 0 ? t.log_k0 : f;
}

// sqrtf(-2 * logf(u1)): the radius of noiser.rs:474.
__device__ __forceinline__ float bm_radius(uint32_t k1, const BmTables& t, const uint32_t* exc) {
    return __builtin_sqrtf(-2.0f * bm_logf(k1, t, exc));
}

// glibc cosf(TAU * k2 * 2^-24), bit-exact (noiser.rs:475-476).
__device__ __forceinline__ float bm_cosf(uint32_t k2, const BmTables& t, const uint32_t* exc) {
    const float th = kTauF * ((float)k2 * 0x1p-24f);
    const double y = cos_f64(th, t.cos_c, t.cos_s, t.cos_thi, t.cos_tlo);
    float g;
    bool danger;
    float f = round_with_danger(y, t.cos_q[k2 >> 16], &g, &danger);
    if (danger && bit_set(exc, k2)) f = g;
    return f;
}

struct NoiseCtx {
    const BmTables* t;     // LDS copy
    const uint32_t* log_exc;
    const uint32_t* cos_exc;
};

// DeterministicNoise::standard_normal (noiser.rs:470-477).
__device__ __forceinline__ float bm_normal(uint64_t& s, const NoiseCtx& c) {
    s = xs64(s);
    const uint32_t k1 = (uint32_t)(s >> 40);
    s = xs64(s);
    const uint32_t k2 = (uint32_t)(s >> 40);
    return bm_radius(k1, *c.t, c.log_exc) * bm_cosf(k2, *c.t, c.cos_exc);
}

// State before the first normal of row j of a stream with s0 = seed | 1.
__device__ __forceinline__ uint64_t row_start_state(uint64_t seed, int32_t j,
                                                     const uint64_t* jump) {
    const uint64_t s0 = seed | 1ull;
    const uint64_t s1 = gf2_apply(jump + (size_t)(j & 15) * 64, s0);
    return gf2_apply(jump + (size_t)(16 + (j >> 4)) * 64, s1);
}

// Seed of member `tid` for one layer key (eggroll.rs:60-65, noiser.rs:495-506).
__device__ __forceinline__ uint64_t member_seed(uint64_t key, int32_t epoch, int32_t noise_reuse,
                                                int32_t tid, float* sign) {
    int32_t te, tt;
    epoch_thread_sign(epoch, tid, noise_reuse, &te, &tt, sign);
    return noise_seed(key, te, tt);
}

}  // namespace hses
