// spiking.hip -- Poisson rate encoding and the LIF scan, HBM-streaming kernels.
//
// Both kernels map one wavefront to 64 consecutive columns of one row: loads
// and stores of a time plane are contiguous across the wave, and the packed
// spike format is one __ballot per (time step, row, 64 columns) written by a
// single lane.
#include "runtime.h"
#include "spike_fmt.h"

namespace hses {

// K(p) = the number of m in [1, 2^23] with RN32(m / D) < p, D = 8388609.
// The reference compares u = ((v >> 9) + 1) / D (f32 division) with p
// (poisson_encode_fused_oxide.rs:44-52); RN32(m / D) is non-decreasing in m,
// so `u < p` is exactly `(v >> 9) < K(p)`.  RN32(q) < p iff q lies below the
// midpoint between p and its predecessor (q = m / D is never exactly that
// dyadic midpoint: D is odd), so K = floor(mid * D), clamped to 2^23.
// mid * D = (pp + p) * (D / 2): the sum (25 significant bits) and its product
// with D / 2 = 4194304.5 (24 bits) are exact in f64.  Branch-free: the value
// computed for p <= 0 or NaN is discarded by the final select.
__device__ __forceinline__ uint32_t poisson_threshold(float p) {
    const float pp = __uint_as_float(__float_as_uint(p) - 1u);  // predecessor (Inf -> FLT_MAX)
    const double t = ((double)pp + (double)p) * 4194304.5;
    const uint32_t k = t >= 8388608.0 ? 8388608u : (uint32_t)t;  // t > 0 and never an integer
    return p > 0.0f ? k : 0u;  // p <= 0 or NaN: never fires
}

template <int FMT>
__global__ __launch_bounds__(256) void k_poisson(const float* __restrict__ p, int64_t p_rows,
                                                 const int32_t* __restrict__ prow, int64_t rows,
                                                 int32_t in_dim, int64_t p_stride, int32_t T,
                                                 uint32_t mix, void* __restrict__ out,
                                                 int64_t out_stride, int64_t plane) {
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
    for (int32_t t = 0; t < T; ++t) {
        x ^= x << 13;
        x ^= x >> 17;
        x ^= x << 5;
        const bool spike = valid && (x >> 9) < K;
        store_spike<FMT>(out, t * plane + row * out_stride, word, col, valid, spike);
    }
}

// Bit-packed Poisson (the SNN input path): one wave per row, looping over the
// row's 64-column words.  For each word the T ballot words are gathered into
// lanes 0..T-1 (v_writelane) and written by one store instruction.
extern "C" __device__ int32_t hses_poisson_writelane(int32_t src, int32_t lane, int32_t old)
    __asm("llvm.amdgcn.writelane.i32");

constexpr int P_ROWS_PER_BLOCK = 4;

// TT: T as a compile-time constant (fully unrolled time loop), or 0 (runtime T).
template <int TT>
__global__ __launch_bounds__(64 * P_ROWS_PER_BLOCK) void k_poisson_bits(
    const float* __restrict__ p, int64_t p_rows, const int32_t* __restrict__ prow, int64_t rows,
    int32_t in_dim, int64_t p_stride, int32_t T_rt, uint32_t mix, uint64_t* __restrict__ out,
    int64_t out_stride, int64_t plane) {
    const int32_t T = TT ? TT : T_rt;
    const int64_t row = (int64_t)blockIdx.x * P_ROWS_PER_BLOCK + (threadIdx.x >> 6);
    const int32_t lane = threadIdx.x & 63;
    if (row >= rows) return;  // whole wave exits together
    const int32_t words = (in_dim + 63) >> 6;
    const int64_t src = prow ? (int64_t)prow[row] : row;
    const bool src_ok = src >= 0 && src < p_rows;
    const float* prow_p = p + (src_ok ? src : 0) * p_stride;
    const uint32_t idx0 = (uint32_t)(row * in_dim);  // flat index of the row's first element
    uint64_t* orow = out + row * out_stride + (int64_t)lane * plane;
    // probabilities of the next word are loaded while the current one is encoded
    float pn = (src_ok && lane < in_dim) ? prow_p[lane] : 0.0f;
    for (int32_t word = 0; word < words; ++word) {
        const int32_t col = word * 64 + lane;
        const float pc = pn;
        const int32_t ncol = col + 64;
        pn = (src_ok && ncol < in_dim) ? prow_p[ncol] : 0.0f;
        const uint32_t K = col < in_dim ? poisson_threshold(pc) : 0u;
        uint32_t x = 1000000007u * (idx0 + (uint32_t)col) + mix + 0x9E3779B9u;
        uint32_t wlo = 0, whi = 0;  // lane t: the word of time step t
#pragma unroll
        for (int32_t t = 0; t < (TT ? TT : 64); ++t) {
            if (!TT && t >= T) break;
            x ^= x << 13;
            x ^= x >> 17;
            x ^= x << 5;
            const uint64_t bits = __ballot((x >> 9) < K);  // K = 0 on invalid lanes
            wlo = (uint32_t)hses_poisson_writelane((int32_t)(uint32_t)bits, t, (int32_t)wlo);
            whi = (uint32_t)hses_poisson_writelane((int32_t)(uint32_t)(bits >> 32), t, (int32_t)whi);
        }
        if (lane < T) orow[word] = ((uint64_t)whi << 32) | wlo;
    }
}

// One stage (distance D <= 8) of the 64 x 64 bit transpose on a 32-bit half:
// partner = lane ^ D by DPP, then lanes with bit D clear keep the bits of
// mask m and take the partner's m bits shifted up by D, lanes with bit D set
// the mirror image.  The rotate wraps only bits the select discards.
template <int D>
__device__ __forceinline__ uint32_t tr_stage(uint32_t w, bool set) {
    constexpr uint32_t m = D == 8 ? 0x00FF00FFu : D == 4 ? 0x0F0F0F0Fu : D == 2 ? 0x33333333u : 0x55555555u;
    uint32_t y;
    if constexpr (D == 1) {
        y = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)w, 0xB1, 0xF, 0xF, false);  // quad_perm 1,0,3,2
    } else if constexpr (D == 2) {
        y = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)w, 0x4E, 0xF, 0xF, false);  // quad_perm 2,3,0,1
    } else {
        // row_shl:D into the lanes with bit D clear, row_shr:D into the others
        constexpr int lo_banks = D == 4 ? 0x5 : 0x3;
        const int t = __builtin_amdgcn_update_dpp((int)w, (int)w, 0x100 + D, 0xF, lo_banks, false);
        y = (uint32_t)__builtin_amdgcn_update_dpp(t, (int)w, 0x110 + D, 0xF, 0xF ^ lo_banks, false);
    }
    const uint32_t keep = set ? ~m : m;
    const uint32_t ys = __builtin_amdgcn_alignbit(y, y, set ? D : 32 - D);
    return (w & keep) | (ys & ~keep);
}

// Transpose of the 64 x 64 bit matrix held one row per lane (lane r: bits
// 0-31 of row r in lo, 32-63 in hi): afterwards lane c holds column c.
// Distance 32 is one cross-half lane swap of lo and hi; distance 16 swaps
// 16-bit halves (byte permutes around a 16-lane swap); distances 8..1 are
// DPP stages.
__device__ __forceinline__ void transpose64(uint32_t& lo, uint32_t& hi, int lane) {
    {
        const auto r = __builtin_amdgcn_permlane32_swap(lo, hi, false, false);
        lo = r[0];
        hi = r[1];
    }
    {
        const uint32_t u = __builtin_amdgcn_perm(hi, lo, 0x05040100u);  // low halves
        const uint32_t v = __builtin_amdgcn_perm(hi, lo, 0x07060302u);  // high halves
        const auto r = __builtin_amdgcn_permlane16_swap(u, v, false, false);
        lo = __builtin_amdgcn_perm(r[1], r[0], 0x05040100u);
        hi = __builtin_amdgcn_perm(r[1], r[0], 0x07060302u);
    }
    lo = tr_stage<8>(lo, lane & 8);
    hi = tr_stage<8>(hi, lane & 8);
    lo = tr_stage<4>(lo, lane & 4);
    hi = tr_stage<4>(hi, lane & 4);
    lo = tr_stage<2>(lo, lane & 2);
    hi = tr_stage<2>(hi, lane & 2);
    lo = tr_stage<1>(lo, lane & 1);
    hi = tr_stage<1>(hi, lane & 1);
}

// Bit-packed Poisson for rows with many p == 0 elements (the SNN input: 70%
// exact zeros).  One wave per row, in three phases over LDS:
//   A. classify: K(p) = 0 never fires, K = 2^23 always fires (pattern of all
//      ones), anything else parks its K in pat[col] and appends col to the
//      row's active list (a ballot and a lane prefix count compact it);
//   B. the active elements only run the xorshift32 stream (T steps each),
//      replacing K in pat[col] with the element's T-bit time pattern;
//   C. spike words: 64 / T consecutive words' patterns form a 64 x 64 bit
//      matrix (lane = element of the word, bit = (word, t)); its transpose,
//      six lane-exchange stages, leaves lane (wi, t) holding word wi of time
//      step t, which it stores.
// Only the zero and saturated elements skip their stream; every stream that
// runs is the one of k_poisson_bits (poisson_encode_fused_oxide.rs:61-106).
template <int T>
__global__ __launch_bounds__(256) void k_poisson_sparse(
    const float* __restrict__ p, int64_t p_rows, const int32_t* __restrict__ prow, int64_t rows,
    int32_t in_dim, int64_t p_stride, uint32_t mix, uint64_t* __restrict__ out, int64_t out_stride,
    int64_t plane, int32_t vec) {
    static_assert(T >= 1 && T <= 32 && (T & (T - 1)) == 0, "T must be a power of two <= 32");
    constexpr int WPT = 64 / T;  // words per 64 x 64 transpose
    extern __shared__ __align__(16) unsigned char psm[];
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int32_t words = (in_dim + 63) >> 6;
    uint32_t* pat = reinterpret_cast<uint32_t*>(psm) + (size_t)wv * (words * 96);
    uint16_t* list = reinterpret_cast<uint16_t*>(pat + words * 64);
    const int64_t row = (int64_t)blockIdx.x * 4 + wv;
    if (row >= rows) return;  // whole wave exits together
    const int64_t src = prow ? (int64_t)prow[row] : row;
    const bool src_ok = src >= 0 && src < p_rows;
    const float* prow_p = p + (src_ok ? src : 0) * p_stride;
    const uint32_t idx0 = (uint32_t)(row * in_dim);
    constexpr uint32_t ALL = T == 32 ? 0xffffffffu : ((1u << T) - 1u);

    // A. classify and compact.  Only the exact zeros and ones are decided here
    // (p <= 0 or NaN: never fires; p >= 1: K = 2^23, every step fires, since
    // RN32(m / D) < 1 for every m <= 2^23); an element with 0 < p < 1 parks the
    // bits of p in its pattern slot and appends its column to the active list,
    // and its threshold K(p) is computed in B.  With 16-byte rows (vec) each lane
    // loads four consecutive columns at once, 256 columns per wave load.
    int32_t cnt = 0;
    auto classify = [&](int32_t col, float pv) -> uint32_t {
        const bool full = pv >= 1.0f, act = pv > 0.0f && pv < 1.0f;
        const uint64_t am = __ballot(act);
        if (act) {
            const int32_t pos = cnt + (int32_t)__builtin_amdgcn_mbcnt_hi(
                                          (uint32_t)(am >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)am, 0u));
            list[pos] = (uint16_t)col;
        }
        cnt += (int32_t)__popcll(am);
        return full ? ALL : (act ? __float_as_uint(pv) : 0u);
    };
    if (vec) {
        const int32_t ncol = words * 64;  // pattern slots of the row (zero past in_dim)
        constexpr int PB = 4;             // 1024 columns of loads in flight
        for (int32_t c0 = 0; c0 < ncol; c0 += 256 * PB) {
            float4 pv[PB];
#pragma unroll
            for (int i = 0; i < PB; ++i) {  // every load in bounds, masked after
                const int32_t col = c0 + 256 * i + 4 * lane;
                pv[i] = reinterpret_cast<const float4*>(prow_p)[(col < in_dim ? col : in_dim - 4) >> 2];
                if (!src_ok || col >= in_dim) pv[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
#pragma unroll
            for (int i = 0; i < PB; ++i) {
                const int32_t col = c0 + 256 * i + 4 * lane;
                if (c0 + 256 * i >= ncol) break;
                uint4 pt;
                pt.x = classify(col, pv[i].x);
                pt.y = classify(col + 1, pv[i].y);
                pt.z = classify(col + 2, pv[i].z);
                pt.w = classify(col + 3, pv[i].w);
                if (col < ncol) *reinterpret_cast<uint4*>(pat + col) = pt;
            }
        }
    } else {
        // a batch of PB words' loads is in flight at once
        constexpr int PB = 16;
        for (int32_t w0 = 0; w0 < words; w0 += PB) {
            float pv[PB];
#pragma unroll
            for (int i = 0; i < PB; ++i) {  // every load in bounds, masked after
                const int32_t col = (w0 + i) * 64 + lane;
                pv[i] = prow_p[col < in_dim ? col : in_dim - 1];
            }
#pragma unroll
            for (int i = 0; i < PB; ++i)
                if (!src_ok || (w0 + i) * 64 + lane >= in_dim) pv[i] = 0.0f;
#pragma unroll
            for (int i = 0; i < PB; ++i) {
                if (w0 + i >= words) break;
                const int32_t col = (w0 + i) * 64 + lane;
                pat[col] = classify(col, pv[i]);
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // B. the streams of the active elements: the exact threshold K(p), then
    // the T steps of the element's xorshift32 stream.  Each step's bit enters
    // at the bottom by one compare and one add-with-carry (pt + pt + carry),
    // and the pattern is bit-reversed at the end.  K = 2^23 (p just below 1)
    // fires every step.
    for (int32_t e = lane; e < cnt; e += 64) {
        const uint32_t col = list[e];
        const uint32_t K = poisson_threshold(__uint_as_float(pat[col]));
        const uint32_t K9 = K << 9;  // (x >> 9) < K  <=>  x < K * 2^9 for K < 2^23
        uint32_t x = 1000000007u * (idx0 + col) + mix + 0x9E3779B9u;
        uint32_t pt = 0;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            x ^= x << 13;
            x ^= x >> 17;
            x ^= x << 5;
            asm("v_cmp_lt_u32 vcc, %1, %2\n\tv_addc_co_u32 %0, vcc, %0, %0, vcc"
                : "+v"(pt)
                : "v"(x), "v"(K9)
                : "vcc");
        }
        pt = __builtin_bitreverse32(pt) >> (32 - T);
        pat[col] = K >= 8388608u ? ALL : pt;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // C. transpose and store
    const int32_t wi = lane / T, t = lane % T;
    uint64_t* orow = out + (int64_t)t * plane + row * out_stride;
    for (int32_t w0 = 0; w0 < words; w0 += WPT) {
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < WPT; ++i) {
            const int32_t wr = w0 + i < words ? w0 + i : words - 1;  // in bounds, masked below
            const uint32_t v = w0 + i < words ? pat[wr * 64 + lane] : 0u;
            if (i * T < 32)
                lo |= v << (i * T);
            else
                hi |= v << (i * T - 32);
        }
        transpose64(lo, hi, lane);
        if (w0 + wi < words) orow[w0 + wi] = ((uint64_t)hi << 32) | lo;
    }
}

static size_t poisson_sparse_lds(int32_t in_dim) {
    const size_t words = (size_t)(in_dim + 63) / 64;
    return 4 * words * 96 * 4;  // 4 waves, each a u32 pattern and a u16 list entry per element
}

// ---- prepared pools ---------------------------------------------------------
//
// A training loop encodes batches gathered from one fixed pool of probability
// rows (accumulate_train.rs:726-735: train_img.select(0, idx), then
// poisson_encode_fused).  k_poisson_sparse classifies every element of every
// gathered row again (its threshold, whether it can fire, the compaction):
// about as many vector instructions as the streams themselves.  A prepared
// pool holds that classification once per pool row:
//   counts  int32 [pool_rows][2]: n_act, n_sat
//   K       u32 [pool_rows][cap]: thresholds K(p) of the active elements
//           (0 < K < 2^23), slots [0, n_act)
//   col     u16 [pool_rows][cap]: their columns in slots [0, n_act); the
//           saturated elements' (K(p) = 2^23: every step fires) in slots
//           [cap - n_sat, cap)
// Elements with K(p) = 0 (p <= 0, NaN, or too small for any u) never fire and
// are left out.  cap = in_dim rounded up to 8 (16-byte aligned rows).
__host__ __device__ constexpr size_t pool_align16(size_t x) { return (x + 15) & ~(size_t)15; }

struct PoolLayout {
    int32_t cap;
    size_t off_k, off_col, bytes;
    __host__ __device__ PoolLayout(int64_t pool_rows, int32_t in_dim) {
        cap = (in_dim + 7) & ~7;
        off_k = pool_align16((size_t)pool_rows * 8);
        off_col = off_k + pool_align16((size_t)pool_rows * cap * 4);
        bytes = off_col + pool_align16((size_t)pool_rows * cap * 2);
    }
};

// One wave per pool row: the row's thresholds, compacted by ballot (active
// from the front, saturated from the back, both in column order).
__global__ __launch_bounds__(256) void k_poisson_pool_prepare(const float* __restrict__ p,
                                                              int64_t pool_rows, int32_t in_dim,
                                                              int64_t p_stride,
                                                              unsigned char* __restrict__ pool) {
    const PoolLayout lay(pool_rows, in_dim);
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= pool_rows) return;  // whole wave exits together
    const float* pr = p + row * p_stride;
    uint32_t* kr = reinterpret_cast<uint32_t*>(pool + lay.off_k) + row * lay.cap;
    uint16_t* cr = reinterpret_cast<uint16_t*>(pool + lay.off_col) + row * lay.cap;
    int32_t na = 0, ns = 0;
    for (int32_t c0 = 0; c0 < in_dim; c0 += 64) {
        const int32_t col = c0 + lane;
        const uint32_t K = col < in_dim ? poisson_threshold(pr[col]) : 0u;
        const bool sat = K >= 8388608u, act = K > 0u && !sat;
        const uint64_t am = __ballot(act), sm = __ballot(sat);
        const uint32_t below_a = __builtin_amdgcn_mbcnt_hi((uint32_t)(am >> 32),
                                                           __builtin_amdgcn_mbcnt_lo((uint32_t)am, 0u));
        const uint32_t below_s = __builtin_amdgcn_mbcnt_hi((uint32_t)(sm >> 32),
                                                           __builtin_amdgcn_mbcnt_lo((uint32_t)sm, 0u));
        if (act) {
            kr[na + (int32_t)below_a] = K;
            cr[na + (int32_t)below_a] = (uint16_t)col;
        }
        if (sat) cr[lay.cap - 1 - (ns + (int32_t)below_s)] = (uint16_t)col;
        na += (int32_t)__popcll(am);
        ns += (int32_t)__popcll(sm);
    }
    if (lane == 0) reinterpret_cast<int2*>(pool)[row] = make_int2(na, ns);
}

// Bit-packed Poisson of rows gathered from a prepared pool: one wave per
// output row and workgroup (3.3 KB of LDS at in_dim 784; no workgroup
// barrier, so a wave starts its next row as soon as it is done).  The row's
// pattern slots in LDS start at zero; the saturated
// columns get the all-ones pattern; each active element runs its xorshift32
// stream (the same stream, seed and compare as k_poisson_sparse's phase B)
// with the next element's column and threshold already loaded; then the
// 64 x 64 bit transposes of k_poisson_sparse's phase C store the words.
template <int T>
__global__ __launch_bounds__(64) void k_poisson_pool(const unsigned char* __restrict__ pool,
                                                      int64_t pool_rows,
                                                      const int32_t* __restrict__ prow,
                                                      int64_t rows, int32_t in_dim, uint32_t mix,
                                                      uint64_t* __restrict__ out,
                                                      int64_t out_stride, int64_t plane) {
    static_assert(T >= 1 && T <= 32 && (T & (T - 1)) == 0, "T must be a power of two <= 32");
    constexpr int WPT = 64 / T;
    constexpr uint32_t ALL = T == 32 ? 0xffffffffu : ((1u << T) - 1u);
    extern __shared__ __align__(16) unsigned char psm[];
    const PoolLayout lay(pool_rows, in_dim);
    const int lane = threadIdx.x;
    const int32_t words = (in_dim + 63) >> 6;
    uint32_t* pat = reinterpret_cast<uint32_t*>(psm);
    const int64_t row = (int64_t)blockIdx.x;
    if (row >= rows) return;  // whole wave exits together
    const int64_t src = prow ? (int64_t)prow[row] : row;
    const bool src_ok = src >= 0 && src < pool_rows;
    const int64_t sr = src_ok ? src : 0;
    const int2 cnt = src_ok ? reinterpret_cast<const int2*>(pool)[sr] : make_int2(0, 0);
    const uint32_t* kr = reinterpret_cast<const uint32_t*>(pool + lay.off_k) + sr * lay.cap;
    const uint16_t* cr = reinterpret_cast<const uint16_t*>(pool + lay.off_col) + sr * lay.cap;
    const uint32_t idx0 = (uint32_t)(row * in_dim);

    for (int32_t i = lane; i < words * 16; i += 64) reinterpret_cast<uint4*>(pat)[i] = make_uint4(0, 0, 0, 0);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    for (int32_t e = lane; e < cnt.y; e += 64) pat[cr[lay.cap - 1 - e]] = ALL;
    // streams of the active elements, the next element's loads in flight
    int32_t e = lane;
    uint32_t col = 0, K9 = 0;
    if (e < cnt.x) {
        col = cr[e];
        K9 = kr[e] << 9;  // (x >> 9) < K  <=>  x < K * 2^9 for K < 2^23
    }
    for (; e < cnt.x; e += 64) {
        const int32_t en = e + 64;
        uint32_t coln = 0, K9n = 0;
        if (en < cnt.x) {
            coln = cr[en];
            K9n = kr[en] << 9;
        }
        uint32_t x = 1000000007u * (idx0 + col) + mix + 0x9E3779B9u;
        uint32_t pt = 0;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            x ^= x << 13;
            x ^= x >> 17;
            x ^= x << 5;
            asm("v_cmp_lt_u32 vcc, %1, %2\n\tv_addc_co_u32 %0, vcc, %0, %0, vcc"
                : "+v"(pt)
                : "v"(x), "v"(K9)
                : "vcc");
        }
        pat[col] = __builtin_bitreverse32(pt) >> (32 - T);
        col = coln;
        K9 = K9n;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    const int32_t wi = lane / T, t = lane % T;
    uint64_t* orow = out + (int64_t)t * plane + row * out_stride;
    for (int32_t w0 = 0; w0 < words; w0 += WPT) {
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < WPT; ++i) {
            const int32_t wr = w0 + i < words ? w0 + i : words - 1;  // in bounds, masked below
            const uint32_t v = w0 + i < words ? pat[wr * 64 + lane] : 0u;
            if (i * T < 32)
                lo |= v << (i * T);
            else
                hi |= v << (i * T - 32);
        }
        transpose64(lo, hi, lane);
        if (w0 + wi < words) orow[w0 + wi] = ((uint64_t)hi << 32) | lo;
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
    // lanes past the row read its last column (discarded): every load is in
    // bounds and unconditional, so a batch of LB steps' loads is in flight at once
    const float* cp = cur + row * cur_stride + (valid ? col : h - 1);
    constexpr int LB = 16;
    for (int32_t t0 = 0; t0 < T; t0 += LB) {
        float cb[LB];
#pragma unroll
        for (int i = 0; i < LB; ++i) cb[i] = cp[(int64_t)min(t0 + i, T - 1) * cplane];
#pragma unroll
        for (int i = 0; i < LB; ++i) {
            const int32_t t = t0 + i;
            if (t >= T) break;  // uniform
            const float c = valid ? cb[i] : 0.0f;
            // snn.rs:61-63: charged = v + ((-v) + c) * leak; each op rounds.
            const float charged = __fadd_rn(v, __fmul_rn(__fadd_rn(-v, c), leak));
            const bool spike = charged >= v_th;
            v = __fmul_rn(charged, __fadd_rn(spike ? -1.0f : -0.0f, 1.0f));
            store_spike<FMT>(spk, t * splane + row * spk_stride, word, col, valid, spike);
        }
    }
    if (valid && v_out) v_out[row * h + col] = v;
}

// The LIF scan with 16-byte loads, for rows of a multiple of 64 columns: a
// dword per lane caps a load stream near half the HBM peak on gfx950, a dwordx4
// per lane does not.  Loads and the per-lane spike stores are non-temporal
// (streamed data, read or written once).  Each 16-lane row of the wave owns one 64-column word
// (lane j of it columns 4j .. 4j+3), so a wave scans four (row, word) items.
// BITS: every lane forms the nibble of its four spikes, shifted to its place in
// the word; ORs over the half-row (quad swaps, half-row mirror) leave the low
// and high 32 bits in lanes 0..7 and 8..15, a row mirror brings the high half
// to lane 0, which stores the word.  The arithmetic is k_lif's, element by
// element, so the outputs are identical.
typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));

template <int FMT>
__global__ __launch_bounds__(256) void k_lif4(const float* __restrict__ cur,
                                              const float* __restrict__ v0, int32_t T, int64_t rows,
                                              int32_t h, int64_t cur_stride, float leak, float v_th,
                                              void* __restrict__ spk, int64_t spk_stride,
                                              float* __restrict__ v_out) {
    const int32_t words = h >> 6;
    const int64_t items = rows * words;
    const int32_t lane = threadIdx.x & 63, g = lane & 15;
    const int64_t item0 = (((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6) * 4;
    if (item0 >= items) return;  // whole wave
    const int64_t it = item0 + (lane >> 4);
    const bool valid = it < items;  // uniform over the 16-lane row
    const int64_t itc = valid ? it : items - 1;
    const int64_t row = itc / words;
    const int32_t word = (int32_t)(itc - row * words);
    const int32_t col = word * 64 + 4 * g;
    float4 v = (valid && v0) ? *reinterpret_cast<const float4*>(v0 + row * h + col)
                             : float4{0.0f, 0.0f, 0.0f, 0.0f};
    const int64_t cplane = rows * cur_stride, splane = rows * spk_stride;
    const float4* cp = reinterpret_cast<const float4*>(cur + row * cur_stride + col);
    const int64_t cp4 = cplane / 4;
    auto step = [&](float& vv, float c) {
        // snn.rs:61-63: charged = v + ((-v) + c) * leak; each op rounds.
        const float charged = __fadd_rn(vv, __fmul_rn(__fadd_rn(-vv, c), leak));
        const bool spike = charged >= v_th;
        vv = __fmul_rn(charged, __fadd_rn(spike ? -1.0f : -0.0f, 1.0f));
        return spike;
    };
    constexpr int LB = 16;
    for (int32_t t0 = 0; t0 < T; t0 += LB) {
        float4 cb[LB];
#pragma unroll
        for (int i = 0; i < LB; ++i) {
            const f32x4v q = __builtin_nontemporal_load(
                reinterpret_cast<const f32x4v*>(cp + (int64_t)min(t0 + i, T - 1) * cp4));
            cb[i] = float4{q.x, q.y, q.z, q.w};
        }
#pragma unroll
        for (int i = 0; i < LB; ++i) {
            const int32_t t = t0 + i;
            if (t >= T) break;  // uniform
            const bool s0 = step(v.x, cb[i].x), s1 = step(v.y, cb[i].y);
            const bool s2 = step(v.z, cb[i].z), s3 = step(v.w, cb[i].w);
            const int64_t base = t * splane + row * spk_stride;
            if constexpr (FMT == HSES_FMT_BITS) {
                const uint32_t nib = (uint32_t)s0 | ((uint32_t)s1 << 1) | ((uint32_t)s2 << 2) |
                                     ((uint32_t)s3 << 3);
                int32_t w = (int32_t)(nib << (4 * (g & 7)));
                w |= __builtin_amdgcn_mov_dpp(w, 0xB1, 0xF, 0xF, true);   // quad_perm 1,0,3,2
                w |= __builtin_amdgcn_mov_dpp(w, 0x4E, 0xF, 0xF, true);   // quad_perm 2,3,0,1
                w |= __builtin_amdgcn_mov_dpp(w, 0x141, 0xF, 0xF, true);  // row_half_mirror
                const int32_t hi = __builtin_amdgcn_mov_dpp(w, 0x140, 0xF, 0xF, true);  // row_mirror
                if (valid && g == 0)
                    static_cast<uint64_t*>(spk)[base + word] = ((uint64_t)(uint32_t)hi << 32) | (uint32_t)w;
            } else if constexpr (FMT == HSES_FMT_F32) {
                if (valid)
                    __builtin_nontemporal_store(
                        f32x4v{s0 ? 1.0f : 0.0f, s1 ? 1.0f : 0.0f, s2 ? 1.0f : 0.0f, s3 ? 1.0f : 0.0f},
                        reinterpret_cast<f32x4v*>(static_cast<float*>(spk) + base + col));
            } else if constexpr (FMT == HSES_FMT_BF16) {
                if (valid)
                    __builtin_nontemporal_store(
                        u32x2v{(s0 ? 0x3f80u : 0u) | (s1 ? 0x3f800000u : 0u),
                               (s2 ? 0x3f80u : 0u) | (s3 ? 0x3f800000u : 0u)},
                        reinterpret_cast<u32x2v*>(static_cast<uint16_t*>(spk) + base + col));
            } else {
                if (valid)
                    __builtin_nontemporal_store(
                        (uint32_t)s0 | ((uint32_t)s1 << 8) | ((uint32_t)s2 << 16) | ((uint32_t)s3 << 24),
                        reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(spk) + base + col));
            }
        }
    }
    if (valid && v_out) *reinterpret_cast<float4*>(v_out + row * h + col) = v;
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

extern "C" int hses_poisson_encode_planes(const float* d_p, int64_t p_rows, const int32_t* d_rows,
                                          int64_t rows, int32_t in_dim, int64_t p_stride, int32_t T,
                                          uint32_t s0, uint32_t s1, uint32_t s2, uint32_t s3,
                                          void* d_out, int32_t fmt, int64_t out_stride,
                                          int64_t out_plane, void* stream) {
    HSES_REQUIRE(rows >= 0 && in_dim >= 0 && T >= 0, "negative size");
    HSES_REQUIRE(fmt >= HSES_FMT_F32 && fmt <= HSES_FMT_BITS, "unknown spike format");
    if (rows == 0 || in_dim == 0 || T == 0) return HSES_OK;
    HSES_REQUIRE(d_p && d_out, "NULL pointer");
    HSES_REQUIRE(p_stride >= in_dim, "p_stride < in_dim");
    HSES_REQUIRE(d_rows || p_rows >= rows, "p_rows < rows without a row index");
    HSES_REQUIRE(rows_layout_ok(fmt_row_units(fmt, in_dim), rows, T, out_stride, out_plane),
                 "output rows overlap (out_stride too small for the format, or time planes overlap)");
    // The reference seeds with the flat index as u32 (poisson_encode_fused_oxide.rs:68-83).
    HSES_REQUIRE(rows * in_dim <= (int64_t)UINT32_MAX, "rows*in_dim exceeds the u32 index range");
    const int64_t blocks = wave_blocks(rows, in_dim);
    HSES_REQUIRE(blocks < (1ll << 31), "grid too large");
    const uint32_t mix = s0 ^ s1 ^ s2 ^ s3;
    hipStream_t s = (hipStream_t)stream;
    switch (fmt) {
        case HSES_FMT_F32:
            hipLaunchKernelGGL(k_poisson<HSES_FMT_F32>, dim3(blocks), dim3(256), 0, s, d_p, p_rows, d_rows,
                               rows, in_dim, p_stride, T, mix, d_out, out_stride, out_plane);
            break;
        case HSES_FMT_BF16:
            hipLaunchKernelGGL(k_poisson<HSES_FMT_BF16>, dim3(blocks), dim3(256), 0, s, d_p, p_rows, d_rows,
                               rows, in_dim, p_stride, T, mix, d_out, out_stride, out_plane);
            break;
        case HSES_FMT_U8:
            hipLaunchKernelGGL(k_poisson<HSES_FMT_U8>, dim3(blocks), dim3(256), 0, s, d_p, p_rows, d_rows,
                               rows, in_dim, p_stride, T, mix, d_out, out_stride, out_plane);
            break;
        default:
            if (T <= 32 && (T & (T - 1)) == 0 && in_dim <= 2048) {
                // zero-skipping kernel: T a power of two, 24 B of LDS per element (48 KiB at 2048)
                const dim3 g((uint32_t)((rows + 3) / 4)), b(256);
                uint64_t* o = static_cast<uint64_t*>(d_out);
                const size_t lds = poisson_sparse_lds(in_dim);
                // rows of whole 16-byte groups: four columns per lane and load
                const int32_t vec = in_dim % 4 == 0 && p_stride % 4 == 0 &&
                                    reinterpret_cast<uintptr_t>(d_p) % 16 == 0;
#define HSES_PSPARSE(TV)                                                                        \
    case TV:                                                                                    \
        hipLaunchKernelGGL(k_poisson_sparse<TV>, g, b, lds, s, d_p, p_rows, d_rows, rows, in_dim, \
                           p_stride, mix, o, out_stride, out_plane, vec);                          \
        break;
                switch (T) {
                    HSES_PSPARSE(1)
                    HSES_PSPARSE(2)
                    HSES_PSPARSE(4)
                    HSES_PSPARSE(8)
                    HSES_PSPARSE(16)
                    HSES_PSPARSE(32)
                }
#undef HSES_PSPARSE
            } else if (T <= 64) {
                const dim3 g((uint32_t)((rows + P_ROWS_PER_BLOCK - 1) / P_ROWS_PER_BLOCK));
                const dim3 b(64 * P_ROWS_PER_BLOCK);
                uint64_t* o = static_cast<uint64_t*>(d_out);
                if (T == 16)
                    hipLaunchKernelGGL(k_poisson_bits<16>, g, b, 0, s, d_p, p_rows, d_rows, rows,
                                       in_dim, p_stride, T, mix, o, out_stride, out_plane);
                else if (T == 8)
                    hipLaunchKernelGGL(k_poisson_bits<8>, g, b, 0, s, d_p, p_rows, d_rows, rows,
                                       in_dim, p_stride, T, mix, o, out_stride, out_plane);
                else
                    hipLaunchKernelGGL(k_poisson_bits<0>, g, b, 0, s, d_p, p_rows, d_rows, rows,
                                       in_dim, p_stride, T, mix, o, out_stride, out_plane);
            }
            else
                hipLaunchKernelGGL(k_poisson<HSES_FMT_BITS>, dim3(blocks), dim3(256), 0, s, d_p, p_rows,
                                   d_rows, rows, in_dim, p_stride, T, mix, d_out, out_stride, out_plane);
            break;
    }
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_poisson_encode(const float* d_p, int64_t p_rows, const int32_t* d_rows, int64_t rows,
                                   int32_t in_dim, int64_t p_stride, int32_t T, uint32_t s0,
                                   uint32_t s1, uint32_t s2, uint32_t s3, void* d_out, int32_t fmt,
                                   int64_t out_stride, void* stream) {
    return hses_poisson_encode_planes(d_p, p_rows, d_rows, rows, in_dim, p_stride, T, s0, s1, s2, s3,
                                      d_out, fmt, out_stride, rows * out_stride, stream);
}

extern "C" size_t hses_poisson_pool_bytes(int64_t pool_rows, int32_t in_dim) {
    if (pool_rows <= 0 || in_dim <= 0 || in_dim > 2048) return 0;
    return PoolLayout(pool_rows, in_dim).bytes;
}

extern "C" int hses_poisson_pool_prepare(const float* d_p, int64_t pool_rows, int32_t in_dim,
                                         int64_t p_stride, void* d_pool, size_t pool_bytes,
                                         void* stream) {
    HSES_REQUIRE(pool_rows >= 0 && in_dim >= 0, "negative size");
    if (pool_rows == 0 || in_dim == 0) return HSES_OK;
    HSES_REQUIRE(in_dim <= 2048, "in_dim > 2048");
    HSES_REQUIRE(d_p && d_pool, "NULL pointer");
    HSES_REQUIRE(p_stride >= in_dim, "p_stride < in_dim");
    HSES_REQUIRE(reinterpret_cast<uintptr_t>(d_pool) % 16 == 0, "pool buffer not 16-byte aligned");
    HSES_REQUIRE(pool_bytes >= PoolLayout(pool_rows, in_dim).bytes,
                 "pool buffer smaller than hses_poisson_pool_bytes");
    const int64_t blocks = (pool_rows + 3) / 4;
    HSES_REQUIRE(blocks < (1ll << 31), "grid too large");
    hipLaunchKernelGGL(k_poisson_pool_prepare, dim3((uint32_t)blocks), dim3(256), 0,
                       (hipStream_t)stream, d_p, pool_rows, in_dim, p_stride,
                       static_cast<unsigned char*>(d_pool));
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_poisson_encode_pool(const void* d_pool, size_t pool_bytes, int64_t pool_rows,
                                        int32_t in_dim, const int32_t* d_rows, int64_t rows,
                                        int32_t T, uint32_t s0, uint32_t s1, uint32_t s2,
                                        uint32_t s3, uint64_t* d_out, int64_t out_stride,
                                        int64_t out_plane, void* stream) {
    HSES_REQUIRE(rows >= 0 && in_dim >= 0 && T >= 0 && pool_rows >= 0, "negative size");
    if (rows == 0 || in_dim == 0 || T == 0) return HSES_OK;
    HSES_REQUIRE(T <= 32 && (T & (T - 1)) == 0, "T must be a power of two <= 32");
    HSES_REQUIRE(in_dim <= 2048, "in_dim > 2048");
    HSES_REQUIRE(d_out && (d_pool || pool_rows == 0), "NULL pointer");
    HSES_REQUIRE(pool_rows == 0 || pool_bytes >= PoolLayout(pool_rows, in_dim).bytes,
                 "pool buffer smaller than hses_poisson_pool_bytes");
    HSES_REQUIRE(reinterpret_cast<uintptr_t>(d_pool) % 16 == 0, "pool buffer not 16-byte aligned");
    HSES_REQUIRE(d_rows || pool_rows >= rows, "pool_rows < rows without a row index");
    HSES_REQUIRE(rows_layout_ok(fmt_row_units(HSES_FMT_BITS, in_dim), rows, T, out_stride, out_plane),
                 "output rows overlap (out_stride too small, or time planes overlap)");
    HSES_REQUIRE(rows * in_dim <= (int64_t)UINT32_MAX, "rows*in_dim exceeds the u32 index range");
    HSES_REQUIRE(rows < (1ll << 31), "grid too large");
    const int64_t blocks = rows;
    const uint32_t mix = s0 ^ s1 ^ s2 ^ s3;
    const size_t lds = (size_t)((in_dim + 63) / 64) * 64 * 4;  // a u32 pattern per slot
    const unsigned char* pl = static_cast<const unsigned char*>(d_pool);
    hipStream_t s = (hipStream_t)stream;
#define HSES_PPOOL(TV)                                                                          \
    case TV:                                                                                    \
        hipLaunchKernelGGL(k_poisson_pool<TV>, dim3((uint32_t)blocks), dim3(64), lds, s, pl,      \
                           pool_rows, d_rows, rows, in_dim, mix, d_out, out_stride, out_plane); \
        break;
    switch (T) {
        HSES_PPOOL(1)
        HSES_PPOOL(2)
        HSES_PPOOL(4)
        HSES_PPOOL(8)
        HSES_PPOOL(16)
        HSES_PPOOL(32)
    }
#undef HSES_PPOOL
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
    // 16-byte loads (k_lif4) when rows are whole 64-column words and every
    // row start keeps the vector accesses aligned
    const auto al = [](const void* q, uintptr_t a) { return reinterpret_cast<uintptr_t>(q) % a == 0; };
    const int64_t ub = fmt_unit_bytes(fmt);
    if (h % 64 == 0 && cur_stride % 4 == 0 && al(d_cur, 16) && al(d_v0, 16) && al(d_v_out, 16) &&
        (fmt == HSES_FMT_BITS || (spk_stride % 4 == 0 && al(d_spikes, 4 * ub)))) {
        const int64_t blocks4 = (rows * (h / 64) + 15) / 16;  // 4 items per wave, 4 waves per block
        switch (fmt) {
            case HSES_FMT_F32:
                hipLaunchKernelGGL(k_lif4<HSES_FMT_F32>, dim3(blocks4), dim3(256), 0, s, d_cur, d_v0, T,
                                   rows, h, cur_stride, leak, v_th, d_spikes, spk_stride, d_v_out);
                break;
            case HSES_FMT_BF16:
                hipLaunchKernelGGL(k_lif4<HSES_FMT_BF16>, dim3(blocks4), dim3(256), 0, s, d_cur, d_v0,
                                   T, rows, h, cur_stride, leak, v_th, d_spikes, spk_stride, d_v_out);
                break;
            case HSES_FMT_U8:
                hipLaunchKernelGGL(k_lif4<HSES_FMT_U8>, dim3(blocks4), dim3(256), 0, s, d_cur, d_v0, T,
                                   rows, h, cur_stride, leak, v_th, d_spikes, spk_stride, d_v_out);
                break;
            default:
                hipLaunchKernelGGL(k_lif4<HSES_FMT_BITS>, dim3(blocks4), dim3(256), 0, s, d_cur, d_v0,
                                   T, rows, h, cur_stride, leak, v_th, d_spikes, spk_stride, d_v_out);
                break;
        }
        HSES_CHECK_HIP(hipGetLastError());
        return HSES_OK;
    }
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
