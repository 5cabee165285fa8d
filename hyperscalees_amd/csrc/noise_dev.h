// noise_dev.h -- device side of the noiser stream (see bm_exact.h).
//
// A factor stream for (layer key, epoch', pair) is the row-major sequence of
// normals of an (rows x L) matrix; normal p consumes xorshift64 states 2p+1
// and 2p+2 after s0 = noise_seed(...) | 1 (noiser.rs:437-490).  Kernels give
// each thread whole rows: the state at the start of row j is
// M^(2Lj) s0 = T1[j/16] (T0[j%16] s0), two GF(2) products with matrices from
// the per-L jump table (each stored as 16 x 16 nibble entries, so a product
// is 16 table reads and XORs), after which the thread steps sequentially.
//
// Normals are produced in batches (bm_normals<G>): the G log and G cos
// evaluations are independent, so their f64 latency overlaps, and every
// exception-bitmap load the batch needs is issued before the first is used.
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

struct NoiseCtx {
    const BmTables* t;     // LDS copy
    const uint32_t* log_exc;
    const uint32_t* cos_exc;
};

// Correctly rounded f32 square root for a positive normal s: hardware
// estimate plus the one-ulp correction from the two residuals.
__device__ __forceinline__ float sqrt_rn(float s) {
    const float r = __builtin_amdgcn_sqrtf(s);
    const float rd = __uint_as_float(__float_as_uint(r) - 1u);
    const float ru = __uint_as_float(__float_as_uint(r) + 1u);
    float q = __builtin_fmaf(-rd, r, s) <= 0.0f ? rd : r;
    q = __builtin_fmaf(-ru, r, s) > 0.0f ? ru : q;
    return q;
}

// glibc logf(max(k1 * 2^-24, 1e-9f)), bit-exact (single value).
__device__ __forceinline__ float bm_logf(uint32_t k1, const BmTables& t, const uint32_t* exc) {
    const double y = log_f64(log_arg(k1), t.log_invc, t.log_logc);
    float f = (float)y;
    if (in_danger(y, t.log_dw[k1 >> kBucketShift]) && ((exc[k1 >> 5] >> (k1 & 31)) & 1u))
        f = other_candidate(f, rem29(y));
    return f;
}

// glibc cosf(TAU * k2 * 2^-24), bit-exact (single value).
__device__ __forceinline__ float bm_cosf(uint32_t k2, const BmTables& t, const uint32_t* exc) {
    const double y = cos_f64(cos_arg(k2), k2, t.cos_c, t.cos_s, t.cos_thi, t.cos_tlo);
    float f = (float)y;
    if (in_danger(y, t.cos_dw[k2 >> kBucketShift]) && ((exc[k2 >> 5] >> (k2 & 31)) & 1u))
        f = other_candidate(f, rem29(y));
    return f;
}

// sqrtf(-2 * logf(u1)): the radius of noiser.rs:474.
__device__ __forceinline__ float bm_radius(uint32_t k1, const BmTables& t, const uint32_t* exc) {
    return sqrt_rn(-2.0f * bm_logf(k1, t, exc));
}

// The 24-bit unit index (x >> 40) of a state, as a 32-bit value.  Written as
// an opaque shift of the high word: otherwise the compiler folds the
// truncation away and converts a 64-bit integer to float (a long sequence).
__device__ __forceinline__ uint32_t unit_index(uint64_t x) {
    uint32_t k;
    asm("v_lshrrev_b32 %0, 8, %1" : "=v"(k) : "v"((uint32_t)(x >> 32)));
    return k;
}

// A batch of G normals in flight.  Stage 1 steps the stream, evaluates log
// and cos in f64, rounds to f32 and issues the exception-bitmap loads of the
// values near a rounding midpoint; stage 2 applies the corrections and forms
// sqrt(-2 log u1) * cos(...).  Running stage 1 of the next batch between the
// two stages of a batch hides the bitmap loads' latency.
template <int G>
struct BmPending {
    float fl[G], fc[G];
    uint32_t rl[G], rc[G];  // remainders: direction of the correction
    uint32_t k1[G], k2[G];
    uint32_t wl[G], wc[G];  // exception words (0 when not in danger)
};

// PIPE: loads issued by every lane (for a pipelined caller, see below);
// otherwise only lanes in danger load (a branch skips the load when none is).
template <int G, bool PIPE>
__device__ __forceinline__ void bm_stage1(uint64_t& s, BmPending<G>& p, const NoiseCtx& c) {
    const BmTables& t = *c.t;
#pragma unroll
    for (int i = 0; i < G; ++i) {
        s = xs64(s);
        p.k1[i] = unit_index(s);
        s = xs64(s);
        p.k2[i] = unit_index(s);
    }
    bool dl[G], dc[G];
#pragma unroll
    for (int i = 0; i < G; ++i) {
        const double yl = log_f64(log_arg(p.k1[i]), t.log_invc, t.log_logc);
        const double yc = cos_f64(cos_arg(p.k2[i]), p.k2[i], t.cos_c, t.cos_s, t.cos_thi, t.cos_tlo);
        p.fl[i] = (float)yl;
        p.fc[i] = (float)yc;
        p.rl[i] = rem29(yl);
        p.rc[i] = rem29(yc);
        dl[i] = in_danger_r(p.rl[i], t.log_dw[p.k1[i] >> kBucketShift]);
        dc[i] = in_danger_r(p.rc[i], t.cos_dw[p.k2[i] >> kBucketShift]);
    }
    if constexpr (PIPE) {
        // Every lane loads (lanes out of danger read the zero word past the
        // bitmap, one shared cache line): no branch and no use of the loaded
        // words before stage 2, so the wait there counts exactly the loads
        // still in flight from the batch issued after this one.
#pragma unroll
        for (int i = 0; i < G; ++i) {
            p.wl[i] = c.log_exc[dl[i] ? p.k1[i] >> 5 : kBitmapWords];
            p.wc[i] = c.cos_exc[dc[i] ? p.k2[i] >> 5 : kBitmapWords];
        }
    } else {
#pragma unroll
        for (int i = 0; i < G; ++i) {
            p.wl[i] = dl[i] ? c.log_exc[p.k1[i] >> 5] : 0u;
            p.wc[i] = dc[i] ? c.cos_exc[p.k2[i] >> 5] : 0u;
        }
    }
}

template <int G>
__device__ __forceinline__ void bm_stage2(const BmPending<G>& p, float* out, const NoiseCtx& c) {
    const BmTables& t = *c.t;
#pragma unroll
    for (int i = 0; i < G; ++i) {
        float fl = p.fl[i], fc = p.fc[i];
        if ((p.wl[i] >> (p.k1[i] & 31)) & 1u) fl = other_candidate(fl, p.rl[i]);
        if ((p.wc[i] >> (p.k2[i] & 31)) & 1u) fc = other_candidate(fc, p.rc[i]);
        out[i] = sqrt_rn(-2.0f * fl) * fc;
    }
}

// G consecutive DeterministicNoise::standard_normal draws (noiser.rs:470-477).
template <int G>
__device__ __forceinline__ void bm_normals(uint64_t& s, float* out, const NoiseCtx& c) {
    BmPending<G> p;
    bm_stage1<G, false>(s, p, c);
    bm_stage2<G>(p, out, c);
}

// One normal (used where a single draw is needed).
__device__ __forceinline__ float bm_normal(uint64_t& s, const NoiseCtx& c) {
    float v;
    bm_normals<1>(s, &v, c);
    return v;
}

// `count` consecutive normals of one stream; sink(i, value) receives normal i.
// Batches of G (4 by default), software-pipelined (stage 1 of batch b+1
// before stage 2 of batch b); a tail of 1..G-1 is drawn singly.  A larger G
// keeps more loads and f64 chains in flight where registers allow.
template <int G = 4, typename Sink>
__device__ __forceinline__ void bm_run(uint64_t& s, int32_t count, const NoiseCtx& c, Sink sink) {
    int32_t i = 0;
    if (count >= G) {
        BmPending<G> p;
        bm_stage1<G, true>(s, p, c);
        for (; i + 2 * G <= count; i += G) {
            BmPending<G> q;
            bm_stage1<G, true>(s, q, c);
            float v[G];
            bm_stage2<G>(p, v, c);
#pragma unroll
            for (int j = 0; j < G; ++j) sink(i + j, v[j]);
            p = q;
        }
        float v[G];
        bm_stage2<G>(p, v, c);
#pragma unroll
        for (int j = 0; j < G; ++j) sink(i + j, v[j]);
        i += G;
    }
    for (; i < count; ++i) sink(i, bm_normal(s, c));
}

// bm_run with the loop unrolled by two, the pending batches p and q taking
// turns, so no pipeline state is copied between iterations (the copies cost
// about 5% of a generator's vector instructions; the unrolled body needs about
// ten more registers, which suits a kernel that only generates).  Stage 1
// still runs batch after batch in stream order: the same normals.
// batch(at, v) receives each batch's G normals [at, at + G) together (at a
// multiple of G), sink(i, value) the tail's.
template <int G = 4, typename Batch, typename Sink>
__device__ __forceinline__ void bm_run2(uint64_t& s, int32_t count, const NoiseCtx& c, Batch batch,
                                        Sink sink) {
    int32_t i = 0;
    auto finish = [&](const BmPending<G>& b, int32_t at) {
        float v[G];
        bm_stage2<G>(b, v, c);
        batch(at, v);
    };
    if (count >= G) {
        BmPending<G> p, q;
        bm_stage1<G, true>(s, p, c);  // p: batch [i, i + G)
        for (; i + 3 * G <= count; i += 2 * G) {
            bm_stage1<G, true>(s, q, c);
            finish(p, i);
            bm_stage1<G, true>(s, p, c);
            finish(q, i + G);
        }
        if (i + 2 * G <= count) {
            bm_stage1<G, true>(s, q, c);
            finish(p, i);
            finish(q, i + G);
            i += 2 * G;
        } else {
            finish(p, i);
            i += G;
        }
    }
    for (; i < count; ++i) sink(i, bm_normal(s, c));
}

// J x over GF(2) for J in nibble form (kJumpNib entries: entry 16 i + v is
// J (v << 4i)), so J x is the XOR of 16 entries, one per nibble of x.
__device__ __forceinline__ uint64_t nib_apply(const uint64_t* tab, uint64_t x) {
    const uint32_t lo = (uint32_t)x, hi = (uint32_t)(x >> 32);
    uint64_t y0 = 0, y1 = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        y0 ^= tab[16 * i + ((lo >> (4 * i)) & 15u)];
        y1 ^= tab[16 * (8 + i) + ((hi >> (4 * i)) & 15u)];
    }
    return y0 ^ y1;
}

// State before the first normal of row j of a stream with s0 = seed | 1:
// T2[j / 256] T1[(j / 16) % 16] T0[j % 16] s0 with the nibble-form matrices
// of the row length's jump-table block (T2 is skipped for j < 256, where it
// is the identity).
__device__ __forceinline__ uint64_t row_start_state(uint64_t seed, int32_t j,
                                                     const uint64_t* jump) {
    const uint64_t s0 = seed | 1ull;
    const uint64_t s1 = nib_apply(jump + (size_t)(j & 15) * kJumpNib, s0);
    uint64_t s2 = nib_apply(jump + (size_t)(16 + ((j >> 4) & 15)) * kJumpNib, s1);
    if (j >= 256) s2 = nib_apply(jump + (size_t)(32 + (j >> 8)) * kJumpNib, s2);
    return s2;
}

// Seed of member `tid` for one layer key (eggroll.rs:60-65, noiser.rs:495-506).
__device__ __forceinline__ uint64_t member_seed(uint64_t key, int32_t epoch, int32_t noise_reuse,
                                                int32_t tid, float* sign) {
    int32_t te, tt;
    epoch_thread_sign(epoch, tid, noise_reuse, &te, &tt, sign);
    return noise_seed(key, te, tt);
}

}  // namespace hses
