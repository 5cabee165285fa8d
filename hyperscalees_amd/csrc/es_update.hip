// es_update.hip -- EggRoll ES gradient  g = scale * sum_m f_m A_m B_m^T.
//
// Reference: _simple_lora_update + _do_update (burn_impl/hyperscalees-noiser/src/eggroll.rs:353-404),
// its chunked/einsum forms (eggroll.rs:579-702, 726-915) and the fused
// pair einsum kernel (burn_impl/hyperscalees-kernels/src/einsum_pair_fused_oxide.rs:94-227).
//
// Members 2p and 2p+1 share pair p's stream with A negated for the odd one
// (eggroll.rs:60-65), so the contraction runs over pairs with weight
// w_p = f_2p - f_2p+1 (a member whose partner lies outside the range keeps
// its own signed weight):  g = scale * sum_p sum_c (w_p Ahat_p[:,c]) B_p[:,c]^T,
// i.e. an (a x b) output with K = pairs * r.
//
// Stage 1: a workgroup owns an output tile and a fixed contiguous range of
// pairs; for each pair it regenerates the tile's rows of Ahat and B into LDS,
// rank-chunk by rank-chunk (each thread continues its own row's stream), and
// accumulates with fp32 MFMA.  The partial tile goes to the workspace.
//   k_es_rows (r >= 32): one thread per generated row.  A tile spans up to 128
//     rows of a and up to 384 columns of b, with blockDim = the tile's row
//     count rounded up to a wave, so every generating thread is busy and a
//     pair's A rows are regenerated once per b tile (C3 fc1: 3 tiles instead
//     of 7).  Rank chunks are double-buffered in LDS (one barrier per chunk)
//     and the generation of the next chunk is interleaved with the MFMAs of
//     the current one.
//   k_es_partial (r < 32): 128x128 tiles, 256 threads; a k-chunk of 32 columns
//     holds 32 / r pairs (the pair weight folded into A at generation), so
//     every thread generates a run of stream rows of one pair per chunk.
// Stage 2 (k_es_reduce): each output element sums its partials in double in
// a fixed order (four split ranges, each in four interleaved sums), scales,
// and stores (or adds).  The split count depends on the problem shape only,
// so the result is independent of the device.
#include <math.h>

#include <type_traits>

#include "mfma.h"
#include "noise_dev.h"
#include "runtime.h"

namespace hses {

constexpr int U_TA = 128, U_TB = 128, U_CW = 32, U_THREADS = 256;
constexpr int U_PITCH = U_CW + 1;  // odd pitch: rows written by consecutive lanes hit distinct banks

struct UpdParams {
    const float* f;
    int32_t n, tid_lo;
    uint64_t key;
    int32_t r;
    float bs;
    int32_t epoch, nreuse, a, b;
    int32_t pair_lo, n_pairs, splits;
    int32_t rc;  // stream rows per generation item (small ranks)
    float* work;
    const float* scale;  // k_es_rows: {S, 1/S} (device)
    const BmTables* tables;
    const uint32_t* log_exc;
    const uint32_t* cos_exc;
    const uint64_t* jump;  // row length r
    // k_es_rows<.., true>: the forward's factor record, pair pair_lo + i's raw
    // normal of stream row j, rank c at rec[(i * r + c) * (a + b) + j]
    const float* rec;
};

__host__ __device__ constexpr size_t align_up16(size_t x) { return (x + 15) & ~(size_t)15; }

__host__ __device__ inline int32_t split_begin(int32_t n_pairs, int32_t splits, int32_t s) {
    return (int32_t)(((int64_t)n_pairs * s) / splits);
}

__global__ __launch_bounds__(U_THREADS) void k_es_partial(UpdParams P) {
    __shared__ BmTables tabs;
    __shared__ float As[U_TA * U_PITCH];
    __shared__ float Bs[U_TB * U_PITCH];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int32_t q0 = blockIdx.x * U_TB, o0 = blockIdx.y * U_TA;
    const int32_t bt = min(U_TB, P.b - q0), at = min(U_TA, P.a - o0);
    const int32_t s = blockIdx.z;
    const int32_t p_begin = P.pair_lo + split_begin(P.n_pairs, P.splits, s);
    const int32_t p_end = P.pair_lo + split_begin(P.n_pairs, P.splits, s + 1);

    load_bm_tables(&tabs, P.tables);
    for (int i = tid; i < U_TA * U_PITCH; i += U_THREADS) As[i] = 0.0f;
    for (int i = tid; i < U_TB * U_PITCH; i += U_THREADS) Bs[i] = 0.0f;
    __syncthreads();
    const NoiseCtx ctx{&tabs, P.log_exc, P.cos_exc};

    // A chunk holds pc = 32 / r pairs (its k-columns: pair-major, then rank
    // column); each generation item is rc consecutive stream rows (rows of one
    // factor) of one pair, A rows first.
    const int32_t r = P.r, rc = P.rc;
    const int32_t pc = U_CW / r;
    const int32_t itemsA = (at + rc - 1) / rc, itemsB = (bt + rc - 1) / rc;
    const int32_t per_pair = itemsA + itemsB;

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0, 0, 0, 0};
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;  // wave quadrant
    const int kg = lane >> 4, li = lane & 15;

    for (int32_t p0 = p_begin; p0 < p_end; p0 += pc) {
        const int32_t np = min(pc, p_end - p0);
        const int32_t kc = np * r;  // k-columns of this chunk
        for (int32_t item = tid; item < np * per_pair; item += U_THREADS) {
            const int32_t pl = item / per_pair, it = item - pl * per_pair;
            const int32_t p = p0 + pl;
            const bool is_a = it < itemsA;
            const int32_t first = (is_a ? it : it - itemsA) * rc;  // local row
            const int32_t nrows = min(rc, (is_a ? at : bt) - first);
            const int32_t srow = is_a ? P.b + o0 + first : q0 + first;  // stream row
            float* dst = is_a ? As : Bs;
            // Pair weight from the members of pair p inside [tid_lo, tid_lo+n).
            const int32_t me = 2 * p - P.tid_lo, mo = me + 1;
            const float fe = (me >= 0 && me < P.n) ? P.f[me] : 0.0f;
            const float fo = (mo >= 0 && mo < P.n) ? P.f[mo] : 0.0f;
            const float w = fe - fo;
            int32_t te, tt;
            float sg;
            epoch_thread_sign(P.epoch, 2 * p, P.nreuse, &te, &tt, &sg);
            uint64_t st = row_start_state(noise_seed(P.key, te, tt), srow, P.jump);
            const float scl = is_a ? P.bs : 1.0f;
            // the item's rows are contiguous in the stream: one run of nrows * r normals
            bm_run(st, nrows * r, ctx, [&](int32_t i, float v) {
                const int32_t row = first + i / r, c = i % r;
                dst[row * U_PITCH + pl * r + c] = is_a ? (v * scl) * w : v;
            });
        }
        // The last k-step reads whole groups of 4 columns: clear the tail.
        const int32_t kc4 = (kc + 3) & ~3;
        for (int32_t i = tid; i < (U_TA + U_TB) * (kc4 - kc); i += U_THREADS) {
            const int32_t row = i / (kc4 - kc), c = kc + i % (kc4 - kc);
            (row < U_TA ? As : Bs)[(row < U_TA ? row : row - U_TA) * U_PITCH + c] = 0.0f;
        }
        __syncthreads();
        // acc += (w Ahat[:, k]) B[:, k]^T over this chunk (k-steps of 4).
        for (int32_t ks = 0; ks < kc; ks += 4) {
            float af[4], bf[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) af[i] = As[(wm + i * 16 + li) * U_PITCH + ks + kg];
#pragma unroll
            for (int j = 0; j < 4; ++j) bf[j] = Bs[(wn + j * 16 + li) * U_PITCH + ks + kg];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = mfma_f32(af[i], bf[j], acc[i][j]);
        }
        __syncthreads();
    }

    // Partial tile -> workspace [s][a][b].
    float* out = P.work + (size_t)s * P.a * P.b;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int col = wn + j * 16 + li;
            if (col >= bt) continue;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int row = wm + i * 16 + 4 * kg + v;
                if (row < at) out[(size_t)(o0 + row) * P.b + q0 + col] = acc[i][j][v];
            }
        }
}

// ---- k_es_rows ---------------------------------------------------------------

constexpr int R_CT = 3;          // 16-column tiles per wave (at most)
constexpr int R_MAXT = 512;      // threads (rows) per workgroup
// LDS row of one rank chunk: the 32 values as fp16 high parts, then the 32 low
// parts, then padding (144 B, so the 16 rows of an operand read by a
// quarter-wave fall on distinct banks).
constexpr int R_HP = 72;

struct RowTiles {
    int32_t at, bt;              // tile extent
    int32_t o_base, q_base;      // origin of blockIdx (0, 0)
};

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma_f16(const uint4& a, const uint4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// x = hi + lo with hi = RN16(x), lo = RN16(x - hi): |x - hi - lo| <= 2^-22 |x|
// for x in fp16's normal range (the operands are scaled into it).
__device__ __forceinline__ void split_f16x4(const float (&x)[4], uint2* hi, uint2* lo) {
    const f16x4 h = __builtin_convertvector((f32x4){x[0], x[1], x[2], x[3]}, f16x4);
    const f32x4 hf = __builtin_convertvector(h, f32x4);
    const f16x4 l = __builtin_convertvector((f32x4){x[0] - hf[0], x[1] - hf[1], x[2] - hf[2],
                                                    x[3] - hf[3]}, f16x4);
    *hi = __builtin_bit_cast(uint2, h);
    *lo = __builtin_bit_cast(uint2, l);
}

// Operand scale S (a power of two) of k_es_rows, and 1/S for k_es_reduce.
// The A operand is S * (w_p * Ahat): |Ahat| <= base_sigma * 6.44 (the largest
// Box-Muller radius, u1 >= 2^-24) and |w_p| <= 2 max|f|, so S puts the largest
// product term near 2^15, inside fp16's range, with the low parts of every
// value far above fp16's underflow relative to it.
__global__ __launch_bounds__(1024) void k_es_scale(const float* __restrict__ f, int32_t n, float bs,
                                                  float* __restrict__ out) {
    __shared__ float red[1024];
    float m = 0.0f;
    for (int32_t i = threadIdx.x; i < n; i += 1024) m = fmaxf(m, fabsf(f[i]));
    red[threadIdx.x] = m;
    __syncthreads();
    for (int w = 512; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + w]);
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const float top = 2.0f * red[0] * fabsf(bs) * 6.5f;  // bound on |w_p * Ahat|
        int e = 0;
        if (top > 0.0f && isfinite(top)) {
            frexpf(32768.0f / top, &e);
            e = min(max(e - 1, -100), 100);  // 2^e <= 2^15 / top
        }
        out[0] = ldexpf(1.0f, e);
        out[1] = ldexpf(1.0f, -e);
    }
}

// NRT: 16-row tiles of a (a tile of at <= 16 * NRT rows); CT: 16-column tiles
// per wave.  Both compile-time, so the MFMA block is branch-free: absent
// tiles of a wave compute on clamped rows and are not stored.
// The contraction runs as fp16 MFMAs on split operands: with x = xh + xl for
// both sides, xh*yh + xh*yl + xl*yh (products exact in the fp32 accumulator)
// differs from x*y by < 2^-20 |x y|, and the partial sums are S times the
// fp32 ones (k_es_reduce divides S out).
// REC: the normals come from the factor record instead of the generator; the
// next item's 32 values of this thread's row are loaded while the MFMAs of
// the current item run and converted after them, so the operands, their
// order and the result are those of the generating form.
template <int NRT, int CT, bool REC>
__global__ __launch_bounds__(R_MAXT) void k_es_rows(UpdParams P, RowTiles G) {
    static_assert(NRT <= 8, "the MFMA row tiles are interleaved with the 8 generation batches");
    extern __shared__ __align__(16) unsigned char smem[];
    BmTables* tabs = reinterpret_cast<BmTables*>(smem);
    const int32_t at = G.at, bt = G.bt, rows = at + bt;
    // the record form draws nothing: no generator tables in LDS
    uint16_t* buf0 = reinterpret_cast<uint16_t*>(smem + (REC ? 0 : align_up16(sizeof(BmTables))));
    // halves per buffer: A rows, B rows, then one row shared by the idle
    // threads (written, never read)
    const int32_t bufsz = (rows + 1) * R_HP;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nw = blockDim.x >> 6;
    const int32_t q0 = G.q_base + blockIdx.x * bt, o0 = G.o_base + blockIdx.y * at;
    const int32_t s = blockIdx.z;
    const int32_t p_begin = P.pair_lo + split_begin(P.n_pairs, P.splits, s);
    const int32_t p_end = P.pair_lo + split_begin(P.n_pairs, P.splits, s + 1);
    const int32_t r = P.r;
    const int32_t chunks = (r + U_CW - 1) / U_CW;

    if constexpr (!REC) load_bm_tables(tabs, P.tables);
    for (int i = tid; i < bufsz; i += blockDim.x)  // two buffers = bufsz words
        reinterpret_cast<uint32_t*>(buf0)[i] = 0u;
    __syncthreads();
    const NoiseCtx ctx{tabs, P.log_exc, P.cos_exc};
    const float S = P.scale[0];

    // This thread's stream row: A rows [0, at) first, then B rows.  Threads
    // past the tile's rows generate a copy of row 0 into one shared spare LDS
    // row (never read), which keeps the generation free of divergent branches
    // and the LDS footprint at the tile's rows.
    const bool is_a = tid < at;
    const int32_t srow = is_a ? P.b + o0 + tid : tid < rows ? q0 + (tid - at) : q0;
    const int32_t grow = min(tid, rows);  // LDS row written by this thread

    // MFMA ownership: column tiles wave, wave + nw, ... (at most CT).
    const int32_t nct = (bt + 15) >> 4;
    const int kg = lane >> 4, li = lane & 15;
    int32_t aoff[NRT], boff[CT];  // LDS offsets (halves) of this lane's operand rows
#pragma unroll
    for (int i = 0; i < NRT; ++i) aoff[i] = min(i * 16 + li, at - 1) * R_HP + kg * 8;
#pragma unroll
    for (int j = 0; j < CT; ++j)
        boff[j] = (at + min(min(wave + j * nw, nct - 1) * 16 + li, bt - 1)) * R_HP + kg * 8;
    f32x4 acc[NRT][CT];
#pragma unroll
    for (int i = 0; i < NRT; ++i)
#pragma unroll
        for (int j = 0; j < CT; ++j) acc[i][j] = f32x4{0, 0, 0, 0};

    // Software pipeline over work items u = (pair, rank chunk): while a wave
    // runs the MFMAs of item u from buffer u & 1 it generates item u + 1 into
    // the other buffer, four normals per MFMA row tile.  The row's stream is
    // consumed four normals at a time through a one-batch look-ahead (pend
    // holds stage 1 of the next four normals), so the bitmap loads of a batch
    // are in flight while the MFMAs and the next batch run.
    const int32_t n_items = (p_end - p_begin) * chunks;
    uint64_t st = 0;
    BmPending<4> pend;
    auto start_pair = [&](int32_t p) {
        int32_t te, tt;
        float sg;
        epoch_thread_sign(P.epoch, 2 * p, P.nreuse, &te, &tt, &sg);
        st = row_start_state(noise_seed(P.key, te, tt), srow, P.jump);
        bm_stage1<4, true>(st, pend, ctx);
    };
    auto pair_weight = [&](int32_t p) {
        const int32_t me = 2 * p - P.tid_lo, mo = me + 1;
        const float fe = (me >= 0 && me < P.n) ? P.f[me] : 0.0f;
        const float fo = (mo >= 0 && mo < P.n) ? P.f[mo] : 0.0f;
        return fe - fo;
    };
    // Normals [c, c + cnt) (cnt <= 4) of a chunk into row `dst`: finish the
    // pending batch and start the next.  A values become S * (w * (v * bs))
    // (the fp32 products of the reference, scaled exactly); B values stay v.
    // Only a row's last batch can be short (r % 4), and the look-ahead past
    // the row's end is discarded (a new pair re-seeds).
    auto gen4 = [&](uint16_t* dst, int32_t c, int32_t cnt, float w) {
        const BmPending<4> cur = pend;
        bm_stage1<4, true>(st, pend, ctx);
        __builtin_amdgcn_sched_barrier(0);  // next batch's loads before this batch's use
        float v[4];
        bm_stage2<4>(cur, v, ctx);
        float x[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = e < cnt ? (is_a ? (v[e] * P.bs) * w * S : v[e]) : 0.0f;
        uint2 hi, lo;
        split_f16x4(x, &hi, &lo);
        *reinterpret_cast<uint2*>(dst + c) = hi;
        *reinterpret_cast<uint2*>(dst + U_CW + c) = lo;
    };
    // Zero columns [c, U_CW) of a short last chunk (r % 32 != 0): the MFMAs
    // read all 32 k of a chunk.
    auto zero_tail = [&](uint16_t* dst, int32_t c) {
        for (; c < U_CW; c += 4) {
            *reinterpret_cast<uint2*>(dst + c) = uint2{0, 0};
            *reinterpret_cast<uint2*>(dst + U_CW + c) = uint2{0, 0};
        }
    };
    // The record form: values of item (p, ch) of this thread's row into a
    // register set, then (iterations later) into the LDS row as gen4 would
    // have.
    float pv[U_CW], pw[U_CW];
    const int64_t rstride = (int64_t)P.a + P.b;  // floats between a row's ranks
    auto load_item = [&](float (&pr)[U_CW], int32_t p, int32_t ch) {
        const float* src = P.rec + ((int64_t)(p - P.pair_lo) * r + ch * U_CW) * rstride + srow;
        const int32_t cn = min(U_CW, r - ch * U_CW);
#pragma unroll
        for (int c = 0; c < U_CW; ++c)
            pr[c] = c < cn ? __builtin_nontemporal_load(src + c * rstride) : 0.0f;  // read once
    };
    auto store_item = [&](const float (&pv)[U_CW], uint16_t* dst, int32_t cn, float w) {
#pragma unroll
        for (int c = 0; c < U_CW; c += 4) {
            float x[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                x[e] = c + e < cn ? (is_a ? (pv[c + e] * P.bs) * w * S : pv[c + e]) : 0.0f;
            uint2 hi, lo;
            split_f16x4(x, &hi, &lo);
            *reinterpret_cast<uint2*>(dst + c) = hi;
            *reinterpret_cast<uint2*>(dst + U_CW + c) = lo;
        }
    };
    if (n_items > 0) {
        uint16_t* dst = buf0 + grow * R_HP;
        const int32_t cn = min(U_CW, r);
        const float w0 = pair_weight(p_begin);
        if constexpr (REC) {
            load_item(pv, p_begin, 0);
            store_item(pv, dst, cn, w0);
        } else {
            start_pair(p_begin);
            for (int32_t c = 0; c < cn; c += 4) gen4(dst, c, min(4, cn - c), w0);
            zero_tail(dst, (cn + 3) & ~3);
        }
    }
    __syncthreads();
    // The MFMAs of item u from buffer X: row tile i, then hook(i) (the
    // generating form draws four normals of the next chunk there: the matrix
    // cores of one wave overlap the generation of the other waves).
    auto mfma_item = [&](const uint16_t* X, auto hook) {
        uint4 bh[CT], bl[CT];
#pragma unroll
        for (int j = 0; j < CT; ++j) {
            bh[j] = *reinterpret_cast<const uint4*>(X + boff[j]);
            bl[j] = *reinterpret_cast<const uint4*>(X + boff[j] + U_CW);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (i < NRT) {
                const uint4 ah = *reinterpret_cast<const uint4*>(X + aoff[i]);
                const uint4 al = *reinterpret_cast<const uint4*>(X + aoff[i] + U_CW);
#pragma unroll
                for (int j = 0; j < CT; ++j) {
                    acc[i][j] = mfma_f16(ah, bh[j], acc[i][j]);
                    acc[i][j] = mfma_f16(ah, bl[j], acc[i][j]);
                    acc[i][j] = mfma_f16(al, bh[j], acc[i][j]);
                }
            }
            hook(i);
        }
    };
    auto item_pc = [&](int32_t v, int32_t* p, int32_t* ch) {
        *p = p_begin + v / chunks;
        *ch = v % chunks;
    };
    if constexpr (REC) {
        // Two register sets take turns (the loop unrolled by two, no copies):
        // item u + 1's values, converted into the LDS after the MFMAs of item
        // u, were loaded at the end of iteration u - 2, so two iterations of
        // MFMAs cover the record's load latency.
        int32_t pl, cl;
        if (n_items > 1) {
            item_pc(1, &pl, &cl);
            load_item(pv, pl, cl);
        }
        if (n_items > 2) {
            item_pc(2, &pl, &cl);
            load_item(pw, pl, cl);
        }
        auto rec_iter = [&](int32_t u, float (&pr)[U_CW]) {
            const bool has_next = u + 1 < n_items;
            int32_t pn = 0, chn = 0;
            if (has_next) item_pc(u + 1, &pn, &chn);
            const int32_t ncn = min(U_CW, r - chn * U_CW);
            const float wn = has_next ? pair_weight(pn) : 0.0f;
            const uint16_t* X = buf0 + (u & 1) * bufsz;
            uint16_t* nxt = buf0 + ((u + 1) & 1) * bufsz + grow * R_HP;
            mfma_item(X, [](int) {});
            if (has_next) store_item(pr, nxt, ncn, wn);
            if (u + 3 < n_items) {
                int32_t p3, c3;
                item_pc(u + 3, &p3, &c3);
                load_item(pr, p3, c3);
            }
            __syncthreads();
        };
        for (int32_t u = 0; u < n_items; u += 2) {
            rec_iter(u, pv);
            if (u + 1 < n_items) rec_iter(u + 1, pw);
        }
    } else {
        for (int32_t u = 0; u < n_items; ++u) {
            const int32_t p = p_begin + u / chunks, ch = u % chunks;
            const bool has_next = u + 1 < n_items;
            const int32_t nch = (ch + 1 == chunks) ? 0 : ch + 1;
            const int32_t ncn = min(U_CW, r - nch * U_CW);
            if (has_next && nch == 0) start_pair(p + 1);
            const float wn = has_next ? pair_weight(nch == 0 ? p + 1 : p) : 0.0f;
            const uint16_t* X = buf0 + (u & 1) * bufsz;
            uint16_t* nxt = buf0 + ((u + 1) & 1) * bufsz + grow * R_HP;
            mfma_item(X, [&](int i) {
                if (has_next && 4 * i < ncn) gen4(nxt, 4 * i, min(4, ncn - 4 * i), wn);
            });
            if (has_next && ncn < U_CW) zero_tail(nxt, (ncn + 3) & ~3);
            __syncthreads();
        }
    }

    // Partial tile -> workspace [s][a][b].
    float* out = P.work + (size_t)s * P.a * P.b;
#pragma unroll
    for (int j = 0; j < CT; ++j) {
        const int32_t ct = wave + j * nw;
        if (ct >= nct) continue;
        const int32_t col = ct * 16 + li;
        if (col >= bt) continue;
#pragma unroll
        for (int i = 0; i < NRT; ++i) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int32_t row = i * 16 + 4 * kg + v;
                if (row < at) out[(size_t)(o0 + row) * P.b + q0 + col] = acc[i][j][v];
            }
        }
    }
}

// 64 output elements per 256-thread block: wave w sums the partials of splits
// [w * splits / 4, (w + 1) * splits / 4) of element 64 * block + lane with four
// interleaved double accumulators, and the four waves' sums are added in wave
// order.  The association is fixed by the shape alone.
// inv_s: 1/S of k_es_rows' scaled partials (a power of two), or NULL.
__global__ __launch_bounds__(256) void k_es_reduce(const float* __restrict__ work, int32_t splits,
                                                   int64_t len, float scale,
                                                   const float* __restrict__ inv_s,
                                                   int32_t accumulate, float* __restrict__ g) {
    __shared__ double part[4][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t e = (int64_t)blockIdx.x * 64 + lane;
    const int64_t ec = e < len ? e : len - 1;  // in bounds; discarded below
    const int32_t k0 = (int32_t)((int64_t)splits * w / 4), k1 = (int32_t)((int64_t)splits * (w + 1) / 4);
    const float* src = work + ec;
    double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
    int32_t k = k0;
    for (; k + 4 <= k1; k += 4) {
        s0 += (double)src[(size_t)k * len];
        s1 += (double)src[(size_t)(k + 1) * len];
        s2 += (double)src[(size_t)(k + 2) * len];
        s3 += (double)src[(size_t)(k + 3) * len];
    }
    for (; k < k1; ++k) s0 += (double)src[(size_t)k * len];
    part[w][lane] = (s0 + s1) + (s2 + s3);
    __syncthreads();
    if (w == 0 && e < len) {
        double s = (part[0][lane] + part[1][lane]) + (part[2][lane] + part[3][lane]);
        if (inv_s) s *= (double)inv_s[0];
        const float v = (float)s * scale;
        g[e] = accumulate ? g[e] + v : v;
    }
}

// g[0, len) = 0 (a kernel rather than hipMemsetAsync, so that callers may
// capture the entry point in a graph).
__global__ __launch_bounds__(256) void k_zero(float* __restrict__ g, int64_t len) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e < len) g[e] = 0.0f;
}

// Split count: ~1024 workgroups in total, at least max(8, 32 / r) pairs (one
// k-chunk) per split, at most 512 splits.
static int32_t es_splits(int32_t a, int32_t b, int32_t n_pairs, int32_t rank) {
    const int64_t tiles = (int64_t)((a + U_TA - 1) / U_TA) * ((b + U_TB - 1) / U_TB);
    int64_t s = std::max<int64_t>(1, 1024 / std::max<int64_t>(tiles, 1));
    s = std::min<int64_t>(s, std::max<int32_t>(1, n_pairs / std::max(8, U_CW / rank)));
    s = std::min<int64_t>(s, 512);
    return (int32_t)std::max<int64_t>(s, 1);
}

// k_es_rows tiling of an (a, b) output: a-tiles of up to 128 rows; b-tiles as
// wide as fits 512 rows per workgroup with at most R_CT column tiles per wave.
static int32_t rows_bt_max(int32_t at) {
    int32_t bt = std::min(384, R_MAXT - at) / 16 * 16;
    while (bt > 16) {
        const int32_t nct = (bt + 15) / 16, nw = (at + bt + 63) / 64;
        if ((nct + nw - 1) / nw <= R_CT) break;
        bt -= 16;
    }
    return bt;
}

static int32_t rows_tiles(int32_t a, int32_t b) {
    int32_t t = 0;
    for (int32_t o0 = 0; o0 < a; o0 += 128) {
        const int32_t at = std::min(128, a - o0), btm = rows_bt_max(at);
        t += (b + btm - 1) / btm;
    }
    return t;
}

// Split count of k_es_rows: about 1024 workgroups over the tiles of at least
// 256 threads, at least 8 pairs per split.  Shape-only, so results do not
// depend on the device.
static int32_t rows_splits(int32_t a, int32_t b, int32_t n_pairs) {
    int32_t big = 0;
    for (int32_t o0 = 0; o0 < a; o0 += 128) {
        const int32_t at = std::min(128, a - o0), btm = rows_bt_max(at);
        big += b / btm;
        if (b % btm && at + b % btm > 256) ++big;
    }
    int64_t s = 1024 / std::max(1, big);
    s = std::min<int64_t>(s, std::max<int32_t>(1, n_pairs / 8));
    return (int32_t)std::max<int64_t>(1, std::min<int64_t>(s, 512));
}

static bool use_rows_kernel(int32_t rank) { return rank >= U_CW; }

static void pair_range(int32_t tid_lo, int32_t n, int32_t* lo, int32_t* cnt) {
    *lo = tid_lo / 2;
    *cnt = (tid_lo + n - 1) / 2 - *lo + 1;
}

}  // namespace hses

using namespace hses;

extern "C" size_t hses_es_update_workspace(int32_t a, int32_t b, int32_t rank, int32_t n) {
    if (a <= 0 || b <= 0 || n <= 0 || rank <= 0) return 0;
    int32_t lo, cnt;
    pair_range(0, n, &lo, &cnt);
    // tid_lo parity can add one pair; size for the larger count.
    const int32_t splits = use_rows_kernel(rank) ? rows_splits(a, b, cnt + 1) : es_splits(a, b, cnt + 1, rank);
    return align_up16((size_t)splits * a * b * sizeof(float)) + 16;  // partials, then {S, 1/S}
}

// The ES update into a caller's partials buffer: d_work of work_bytes, or,
// with scratch_cap > 0, at most scratch_cap bytes of it (the split count is
// lowered until the partials fit).
static int es_update_impl(const float* d_f, int32_t n, int32_t tid_lo, uint64_t key, int32_t rank,
                          float sigma, int32_t epoch, int32_t noise_reuse, int32_t a, int32_t b,
                          float scale, int32_t accumulate, float* d_grad, void* d_work,
                          size_t work_bytes, size_t scratch_cap, DeviceState* st,
                          hipStream_t s, const float* rec = nullptr) {
    UpdParams P{};
    int32_t pair_lo, n_pairs;
    pair_range(tid_lo, n, &pair_lo, &n_pairs);
    const bool empty = n == 0 || rank == 0 || sigma == 0.0f;
    const bool rows_k = use_rows_kernel(rank);
    P.splits = empty ? 1 : rows_k ? rows_splits(a, b, n_pairs) : es_splits(a, b, n_pairs, rank);
    const size_t elems = (size_t)a * b;
    if (scratch_cap) {
        const size_t fit = (scratch_cap - 16) / (elems * sizeof(float));
        if (fit < 1)
            return set_error(HSES_ERR_INVALID_ARG, "a * b exceeds the fixed scratch of the "
                                                   "allocation-free ES update");
        P.splits = (int32_t)std::min<size_t>((size_t)P.splits, fit);
    }
    const size_t part_bytes = align_up16((size_t)P.splits * elems * sizeof(float));
    const size_t need = part_bytes + 16;
    if (!empty) {
        HSES_REQUIRE(d_f, "fitness is NULL");
        HSES_REQUIRE(d_work && work_bytes >= need, "workspace too small");
    }
    int rc;
    if (empty) {
        if (!accumulate) {
            const int64_t len = (int64_t)a * b;
            hipLaunchKernelGGL(k_zero, dim3((uint32_t)((len + 255) / 256)), dim3(256), 0, s,
                               d_grad, len);
            HSES_CHECK_HIP(hipGetLastError());
        }
        return HSES_OK;
    }
    P.f = d_f;
    P.n = n;
    P.tid_lo = tid_lo;
    P.key = key;
    P.r = rank;
    P.bs = sigma / sqrtf((float)rank);  // eggroll.rs:365
    P.epoch = epoch;
    P.nreuse = noise_reuse;
    P.a = a;
    P.b = b;
    P.pair_lo = pair_lo;
    P.n_pairs = n_pairs;
    P.rc = rank >= U_CW ? 1 : std::max(1, U_CW / rank);
    P.work = static_cast<float*>(d_work);
    float* d_scale = reinterpret_cast<float*>(static_cast<char*>(d_work) + part_bytes);
    P.scale = d_scale;
    P.tables = st->d_tables;
    P.log_exc = st->d_log_exc;
    P.cos_exc = st->d_cos_exc;
    P.rec = rec;
    if (rec) {
        HSES_REQUIRE(rows_k, "the factor record update needs rank >= 32");
    } else {
        rc = get_jump_table(st, rank, (int64_t)a + b, &P.jump);
        if (rc) return rc;
    }
    if (rows_k) {
        hipLaunchKernelGGL(k_es_scale, dim3(1), dim3(1024), 0, s, P.f, n, P.bs, d_scale);
        HSES_CHECK_HIP(hipGetLastError());
        // One launch per (a-tile, full / remainder b-tile) group.
        for (int32_t o0 = 0; o0 < a; o0 += 128) {
            const int32_t at = std::min(128, a - o0), btm = rows_bt_max(at);
            const int32_t nfull = b / btm, rem = b % btm;
            for (int g = 0; g < 2; ++g) {
                const int32_t bt = g == 0 ? btm : rem, cnt = g == 0 ? nfull : (rem ? 1 : 0);
                if (cnt == 0) continue;
                RowTiles G{at, bt, o0, g == 0 ? 0 : nfull * btm};
                const int32_t threads = (at + bt + 63) / 64 * 64;
                const size_t lds = (rec ? 0 : align_up16(sizeof(BmTables))) +
                                   (size_t)2 * (at + bt + 1) * R_HP * 2;
                const int32_t nw = threads / 64, nct = (bt + 15) / 16;
                const int32_t ct = (nct + nw - 1) / nw;
                auto launch = [&](auto kern) -> int {
                    if (lds > 64 * 1024)
                        HSES_CHECK_HIP(hipFuncSetAttribute(
                            (const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
                    hipLaunchKernelGGL(kern, dim3(cnt, 1, P.splits), dim3(threads), lds, s, P, G);
                    HSES_CHECK_HIP(hipGetLastError());
                    return HSES_OK;
                };
                auto by_src = [&](auto recc) -> int {
                    constexpr bool RC = decltype(recc)::value;
                    if (at <= 16)
                        return ct == 1 ? launch(k_es_rows<1, 1, RC>)
                               : ct == 2 ? launch(k_es_rows<1, 2, RC>) : launch(k_es_rows<1, 3, RC>);
                    return ct == 1 ? launch(k_es_rows<8, 1, RC>)
                           : ct == 2 ? launch(k_es_rows<8, 2, RC>) : launch(k_es_rows<8, 3, RC>);
                };
                const int lrc = rec ? by_src(std::true_type{}) : by_src(std::false_type{});
                if (lrc) return lrc;
            }
        }
    } else {
        dim3 grid((b + U_TB - 1) / U_TB, (a + U_TA - 1) / U_TA, P.splits);
        hipLaunchKernelGGL(k_es_partial, grid, dim3(U_THREADS), 0, s, P);
        HSES_CHECK_HIP(hipGetLastError());
    }
    const int64_t len = (int64_t)a * b;
    hipLaunchKernelGGL(k_es_reduce, dim3((uint32_t)((len + 63) / 64)), dim3(256), 0, s, P.work,
                       P.splits, len, scale, rows_k ? d_scale + 1 : nullptr, accumulate, d_grad);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

static int es_update_check(int32_t n, int32_t tid_lo, int32_t rank, int32_t noise_reuse, int32_t a,
                           int32_t b, const float* d_grad) {
    HSES_REQUIRE(n >= 0 && a >= 1 && b >= 1 && rank >= 0, "bad sizes");
    HSES_REQUIRE(noise_reuse >= 0, "noise_reuse must be >= 0");
    HSES_REQUIRE(tid_lo >= 0 && (int64_t)tid_lo + n - 1 <= INT32_MAX, "thread id range");
    HSES_REQUIRE(d_grad, "grad is NULL");
    return HSES_OK;
}

extern "C" int hses_es_update(const float* d_f, int32_t n, int32_t tid_lo, uint64_t key,
                              int32_t rank, float sigma, int32_t epoch, int32_t noise_reuse,
                              int32_t a, int32_t b, float scale, int32_t accumulate, float* d_grad,
                              void* d_work, size_t work_bytes, void* stream) {
    int rc = es_update_check(n, tid_lo, rank, noise_reuse, a, b, d_grad);
    if (rc) return rc;
    const bool empty = n == 0 || rank == 0 || sigma == 0.0f;
    if (!empty) {
        int32_t lo, cnt;
        pair_range(tid_lo, n, &lo, &cnt);
        const int32_t splits = use_rows_kernel(rank) ? rows_splits(a, b, cnt)
                                                     : es_splits(a, b, cnt, rank);
        HSES_REQUIRE(d_f, "fitness is NULL");
        HSES_REQUIRE(d_work && work_bytes >= align_up16((size_t)splits * a * b * sizeof(float)) + 16,
                     "workspace too small");
    }
    DeviceState* st;
    rc = get_state(&st);
    if (rc) return rc;
    return es_update_impl(d_f, n, tid_lo, key, rank, sigma, epoch, noise_reuse, a, b, scale,
                          accumulate, d_grad, d_work, work_bytes, 0, st, (hipStream_t)stream);
}

// The ES update from the forward's factor record (hses_perturbed_linear_rec /
// hses_perturbed_linear_lif_rec with the same tid_lo and n): the same
// operands, tiles and order as hses_es_update, so the same result, without
// drawing the normals again.
extern "C" int hses_es_update_rec(const float* d_f, int32_t n, int32_t tid_lo, const float* d_rec,
                                  size_t rec_bytes, int32_t rank, float sigma, int32_t a,
                                  int32_t b, float scale, int32_t accumulate, float* d_grad,
                                  void* d_work, size_t work_bytes, void* stream) {
    int rc = es_update_check(n, tid_lo, rank, 0, a, b, d_grad);
    if (rc) return rc;
    const bool empty = n == 0 || rank == 0 || sigma == 0.0f;
    if (!empty) {
        HSES_REQUIRE(rank >= 32, "the factor record update needs rank >= 32");
        HSES_REQUIRE(d_rec, "factor record is NULL");
        int32_t lo, cnt;
        pair_range(tid_lo, n, &lo, &cnt);
        HSES_REQUIRE(rec_bytes >= (size_t)cnt * (size_t)(a + b) * rank * sizeof(float),
                     "factor record smaller than hses_factor_record_bytes");
        HSES_REQUIRE(d_f, "fitness is NULL");
        HSES_REQUIRE(d_work && work_bytes >= align_up16((size_t)rows_splits(a, b, cnt) * a * b *
                                                        sizeof(float)) + 16,
                     "workspace too small");
    }
    DeviceState* st;
    rc = get_state(&st);
    if (rc) return rc;
    return es_update_impl(d_f, n, tid_lo, 0, rank, sigma, 0, 0, a, b, scale, accumulate, d_grad,
                          d_work, work_bytes, 0, st, (hipStream_t)stream, d_rec);
}

// ---- the allocation-free variant ---------------------------------------------
//
// The split-K partials and the operand scale live in this file-scope device
// array instead of a caller workspace.  Each device holds its own copy for
// the life of the process; its address on a device is looked up once, at
// hses_init, and kept in that device's state (the array's name in host code is
// not a device address).  Every call on a device shares the array, so calls
// that overlap on one device (other streams, other threads) race.  Nothing in
// it has to start at zero: every split stores its whole partial tile and the
// scale kernel stores both words it owns.
namespace hses {

static __device__ __align__(256) unsigned char scratch[kEsScratchBytes];

int es_scratch_setup(DeviceState* st) {
    void* ptr = nullptr;
    HSES_CHECK_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    st->es_scratch = ptr;
    return HSES_OK;
}

}  // namespace hses

extern "C" int hses_es_update_noalloc(const float* d_f, int32_t n, int32_t tid_lo, uint64_t key,
                                      int32_t rank, float sigma, int32_t epoch,
                                      int32_t noise_reuse, int32_t a, int32_t b, float scale,
                                      int32_t accumulate, float* d_grad, void* stream) {
    int rc = es_update_check(n, tid_lo, rank, noise_reuse, a, b, d_grad);
    if (rc) return rc;
    HSES_REQUIRE((size_t)a * b * sizeof(float) + 16 <= kEsScratchBytes,
                 "a * b exceeds the fixed scratch of the allocation-free ES update "
                 "(at most (kEsScratchBytes - 16) / 4 elements)");
    DeviceState* st;
    rc = get_state(&st);
    if (rc) return rc;
    HSES_REQUIRE(st->es_scratch, "scratch address of this device is missing");
    return es_update_impl(d_f, n, tid_lo, key, rank, sigma, epoch, noise_reuse, a, b, scale,
                          accumulate, d_grad, st->es_scratch, kEsScratchBytes, kEsScratchBytes, st,
                          (hipStream_t)stream);
}
