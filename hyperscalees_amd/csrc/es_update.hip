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
// Stage 1 (k_es_partial): grid = (b tiles, a tiles, splits).  A workgroup owns
// a 128x128 output tile and a fixed contiguous range of pairs; for each pair it
// regenerates the tile's rows of Ahat and B into LDS, rank-chunk by
// rank-chunk (each thread continues its own row's stream), and accumulates
// with fp32 MFMA.  The partial tile goes to the workspace.
// Stage 2 (k_es_reduce): each output element sums its partials in split
// order in double, scales, and stores (or adds).  The split count depends on
// the problem shape only, so the result is independent of the device.
#include <math.h>

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
    const BmTables* tables;
    const uint32_t* log_exc;
    const uint32_t* cos_exc;
    const uint64_t* jump;  // row length r
};

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

    // Generation items: RC consecutive stream rows each; A rows first.
    const int32_t r = P.r, rc = P.rc;
    const int32_t itemsA = (at + rc - 1) / rc, itemsB = (bt + rc - 1) / rc;
    const bool has_item = tid < itemsA + itemsB;
    const bool is_a = tid < itemsA;
    const int32_t first = is_a ? tid * rc : (tid - itemsA) * rc;       // local row
    const int32_t nrows = has_item ? min(rc, (is_a ? at : bt) - first) : 0;
    const int32_t srow = is_a ? P.b + o0 + first : q0 + first;          // stream row
    float* dst = is_a ? As : Bs;
    const int32_t cw = min(r, U_CW);
    const int32_t chunks = (r + U_CW - 1) / U_CW;

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0, 0, 0, 0};
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;  // wave quadrant
    const int kg = lane >> 4, li = lane & 15;

    for (int32_t p = p_begin; p < p_end; ++p) {
        // Pair weight from the members of pair p inside [tid_lo, tid_lo+n).
        const int32_t me = 2 * p - P.tid_lo, mo = me + 1;
        const float fe = (me >= 0 && me < P.n) ? P.f[me] : 0.0f;
        const float fo = (mo >= 0 && mo < P.n) ? P.f[mo] : 0.0f;
        const float w = fe - fo;
        uint64_t st = 0;
        if (has_item) {
            int32_t te, tt;
            float sg;
            epoch_thread_sign(P.epoch, 2 * p, P.nreuse, &te, &tt, &sg);
            st = row_start_state(noise_seed(P.key, te, tt), srow, P.jump);
        }
        for (int32_t ch = 0; ch < chunks; ++ch) {
            const int32_t c0 = ch * U_CW;
            const int32_t cn = min(cw, r - c0);
            // rc > 1 only when r <= 16 (one chunk): the item's rows are contiguous
            // in the stream, so one run of nrows * r normals covers them.
            const float scl = is_a ? P.bs : 1.0f;
            bm_run(st, nrows * cn, ctx, [&](int32_t i, float v) {
                const int32_t row = first + i / cn, c = i % cn;
                dst[row * U_PITCH + c] = is_a ? v * scl : v;
            });
            // The last k-step reads whole groups of 4 columns: clear the tail.
            for (int32_t i = 0; i < nrows; ++i)
                for (int32_t c = cn; c < ((cn + 3) & ~3); ++c) dst[(first + i) * U_PITCH + c] = 0.0f;
            __syncthreads();
            // acc += (w * Ahat[:, c]) B[:, c]^T over this chunk (k-steps of 4).
            for (int32_t ks = 0; ks < cn; ks += 4) {
                float af[4], bf[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) af[i] = w * As[(wm + i * 16 + li) * U_PITCH + ks + kg];
#pragma unroll
                for (int j = 0; j < 4; ++j) bf[j] = Bs[(wn + j * 16 + li) * U_PITCH + ks + kg];
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[i][j] = mfma_f32(af[i], bf[j], acc[i][j]);
            }
            __syncthreads();
        }
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

__global__ void k_es_reduce(const float* __restrict__ work, int32_t splits, int64_t len, float scale,
                            int32_t accumulate, float* __restrict__ g) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= len) return;
    double s = 0.0;
    for (int32_t k = 0; k < splits; ++k) s += (double)work[(size_t)k * len + e];
    const float v = (float)s * scale;
    g[e] = accumulate ? g[e] + v : v;
}

// Split count: ~1024 workgroups in total, at least 8 pairs per split, at most 512 splits.
static int32_t es_splits(int32_t a, int32_t b, int32_t n_pairs) {
    const int64_t tiles = (int64_t)((a + U_TA - 1) / U_TA) * ((b + U_TB - 1) / U_TB);
    int64_t s = std::max<int64_t>(1, 1024 / std::max<int64_t>(tiles, 1));
    s = std::min<int64_t>(s, std::max<int32_t>(1, n_pairs / 8));
    s = std::min<int64_t>(s, 512);
    return (int32_t)std::max<int64_t>(s, 1);
}

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
    return (size_t)es_splits(a, b, cnt + 1) * a * b * sizeof(float);
}

extern "C" int hses_es_update(const float* d_f, int32_t n, int32_t tid_lo, uint64_t key,
                              int32_t rank, float sigma, int32_t epoch, int32_t noise_reuse,
                              int32_t a, int32_t b, float scale, int32_t accumulate, float* d_grad,
                              void* d_work, size_t work_bytes, void* stream) {
    HSES_REQUIRE(n >= 0 && a >= 1 && b >= 1 && rank >= 0, "bad sizes");
    HSES_REQUIRE(noise_reuse >= 0, "noise_reuse must be >= 0");
    HSES_REQUIRE(tid_lo >= 0 && (int64_t)tid_lo + n - 1 <= INT32_MAX, "thread id range");
    HSES_REQUIRE(d_grad, "grad is NULL");
    UpdParams P{};
    int32_t pair_lo, n_pairs;
    pair_range(tid_lo, n, &pair_lo, &n_pairs);
    const bool empty = n == 0 || rank == 0 || sigma == 0.0f;
    P.splits = empty ? 1 : es_splits(a, b, n_pairs);
    const size_t need = (size_t)P.splits * a * b * sizeof(float);
    if (!empty) {
        HSES_REQUIRE(d_f, "fitness is NULL");
        HSES_REQUIRE(d_work && work_bytes >= need, "workspace too small");
    }
    DeviceState* st;
    int rc = get_state(&st);
    if (rc) return rc;
    hipStream_t s = (hipStream_t)stream;
    if (empty) {
        if (!accumulate) HSES_CHECK_HIP(hipMemsetAsync(d_grad, 0, sizeof(float) * a * b, s));
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
    // Items must cover a tile's rows with the block's threads.
    const int32_t items = (U_TA + P.rc - 1) / P.rc + (U_TB + P.rc - 1) / P.rc;
    if (items > U_THREADS || (P.rc > 1 && rank > U_CW))
        return set_error(HSES_ERR_INTERNAL, "es_update tiling");
    P.work = static_cast<float*>(d_work);
    P.tables = st->d_tables;
    P.log_exc = st->d_log_exc;
    P.cos_exc = st->d_cos_exc;
    rc = get_jump_table(st, rank, (int64_t)a + b, &P.jump);
    if (rc) return rc;
    dim3 grid((b + U_TB - 1) / U_TB, (a + U_TA - 1) / U_TA, P.splits);
    hipLaunchKernelGGL(k_es_partial, grid, dim3(U_THREADS), 0, s, P);
    HSES_CHECK_HIP(hipGetLastError());
    const int64_t len = (int64_t)a * b;
    hipLaunchKernelGGL(k_es_reduce, dim3((uint32_t)((len + 255) / 256)), dim3(256), 0, s, P.work,
                       P.splits, len, scale, accumulate, d_grad);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}
