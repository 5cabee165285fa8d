// noise.hip -- factor materialisation (test mode) and Box-Muller evaluation.
//
// The hot-path kernels (linear.hip, es_update.hip) generate factors in-kernel
// and never write them to HBM; the entry points here exist to check the
// stream bit for bit against the reference layout (eggroll.rs:116-227) and to
// serve get_nonlora_update_params (eggroll.rs:312-324).
#include "noise_dev.h"
#include "runtime.h"

namespace hses {

__global__ __launch_bounds__(256) void k_bm_eval(uint32_t k_lo, uint32_t n, float* lg, float* rad, float* cs,
                          const BmTables* gt, const uint32_t* le, const uint32_t* ce) {
    __shared__ BmTables t;
    load_bm_tables(&t, gt);
    __syncthreads();
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const uint32_t k = k_lo + i;
        if (lg || rad) {
            const float L = bm_logf(k, t, le);
            if (lg) lg[i] = L;
            if (rad) rad[i] = sqrt_rn(-2.0f * L);
        }
        if (cs) cs[i] = bm_cosf(k, t, ce);
    }
}

// One thread per (member, stream row).  Stream rows [0, b) are B rows, rows
// [b, a+b) are A rows scaled by sign*base_sigma (eggroll.rs:86-103).  With
// b == 0 it writes a dense (a, L) noise block instead
// (get_nonlora_update_params: all rows scaled), and with `base` the member's
// perturbed parameter base + noise (get_noisy_standard_impl, eggroll.rs:480-503).
__global__ __launch_bounds__(256) void k_stream_rows(float bs, uint64_t key, int32_t L, int32_t epoch, int32_t nreuse,
                              int32_t tid_lo, const int32_t* tids, int32_t n, int32_t a, int32_t b,
                              int32_t blocks_per_member, float* A, float* B,
                              const BmTables* gt, const uint32_t* le, const uint32_t* ce,
                              const uint64_t* jump, const float* base) {
    __shared__ BmTables t;
    load_bm_tables(&t, gt);
    __syncthreads();
    const int32_t m = blockIdx.x / blocks_per_member;
    const int32_t j = (blockIdx.x % blocks_per_member) * blockDim.x + threadIdx.x;
    if (m >= n || j >= a + b) return;
    const int32_t tid = tids ? tids[m] : tid_lo + m;
    float sign;
    const uint64_t seed = member_seed(key, epoch, nreuse, tid, &sign);
    uint64_t s = row_start_state(seed, j, jump);
    const NoiseCtx ctx{&t, le, ce};
    if (j < b) {
        float* dst = B + ((int64_t)m * b + j) * L;
        bm_run(s, L, ctx, [&](int32_t c, float v) { dst[c] = v; });
    } else if (!base) {
        const float sc = sign * bs;
        float* dst = A + ((int64_t)m * a + (j - b)) * L;
        bm_run(s, L, ctx, [&](int32_t c, float v) { dst[c] = v * sc; });
    } else {
        const float sc = sign * bs;
        float* dst = A + ((int64_t)m * a + (j - b)) * L;
        const float* src = base + (int64_t)(j - b) * L;
        bm_run(s, L, ctx, [&](int32_t c, float v) { dst[c] = src[c] + v * sc; });
    }
}

// _simple_full_update (eggroll.rs:331-350), split-K stage 1.  A thread owns a
// chunk of kFullLc consecutive elements of the dense (a, b) block (normals
// [c kFullLc, (c+1) kFullLc) of every member's stream) and, for the pairs of
// its split, adds each member's f32 term (normal * (sign sigma)) * f in double
// in pair order.  The two members of a pair share one stream (the odd one's
// term is the negated product); a member outside [tid_lo, tid_lo + n) adds
// nothing.  Partials are double, indexed part[split * E + element].
constexpr int kFullLc = 32;
constexpr int kFullThreads = 64;
__global__ __launch_bounds__(kFullThreads) void k_full_partial(
        const float* __restrict__ f, int32_t n, int32_t tid_lo, uint64_t key, float sigma,
        int32_t epoch, int32_t nreuse, int64_t E, int32_t chunks, int32_t pair_lo,
        int32_t n_pairs, int32_t splits, double* __restrict__ part, const BmTables* gt,
        const uint32_t* le, const uint32_t* ce, const uint64_t* jump) {
    __shared__ BmTables t;
    __shared__ double acc[kFullLc][kFullThreads];
    load_bm_tables(&t, gt);
    for (int i = 0; i < kFullLc; ++i) acc[i][threadIdx.x] = 0.0;
    __syncthreads();
    const int32_t c = blockIdx.x * kFullThreads + threadIdx.x;
    const int32_t sp = blockIdx.y;
    if (c >= chunks) return;
    const int32_t p0 = pair_lo + (int32_t)(((int64_t)n_pairs * sp) / splits);
    const int32_t p1 = pair_lo + (int32_t)(((int64_t)n_pairs * (sp + 1)) / splits);
    const int32_t cnt = (int32_t)min<int64_t>(kFullLc, E - (int64_t)c * kFullLc);
    const NoiseCtx ctx{&t, le, ce};
    const int32_t te = nreuse == 0 ? 0 : epoch / nreuse;
    for (int32_t p = p0; p < p1; ++p) {
        const int32_t me = 2 * p - tid_lo, mo = me + 1;
        const bool he = me >= 0 && me < n, ho = mo >= 0 && mo < n;
        const float fe = he ? f[me] : 0.0f, fo = ho ? f[mo] : 0.0f;
        uint64_t s = row_start_state(noise_seed(key, te, p), c, jump);
        bm_run(s, cnt, ctx, [&](int32_t i, float v) {
            const float up = v * sigma;  // the even member's noise; the odd one's is -up
            double d = 0.0;
            if (he) d += (double)(up * fe);
            if (ho) d -= (double)(up * fo);
            acc[i][threadIdx.x] += d;
        });
    }
    double* dst = part + (int64_t)sp * E + (int64_t)c * kFullLc;
    for (int32_t i = 0; i < cnt; ++i) dst[i] = acc[i][threadIdx.x];
}

// Stage 2: g[e] = (f32 of the split partials summed in split order) * scale
// (or added to g with accumulate).
__global__ __launch_bounds__(256) void k_full_reduce(const double* __restrict__ part, int32_t splits,
                                                     int64_t E, float scale, int32_t accumulate,
                                                     float* __restrict__ g) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= E) return;
    double s = 0.0;
    for (int32_t k = 0; k < splits; ++k) s += part[(int64_t)k * E + e];
    const float v = splits ? (float)s * scale : 0.0f;
    g[e] = accumulate ? g[e] + v : v;
}

static int32_t full_splits(int32_t chunks, int32_t n_pairs) {
    int64_t s = std::max<int64_t>(1, 4096 / std::max(1, chunks));
    s = std::min<int64_t>(s, std::max(1, n_pairs));
    return (int32_t)std::min<int64_t>(s, 1024);
}

}  // namespace hses

using namespace hses;

extern "C" int hses_bm_eval(uint32_t k_lo, uint32_t n, float* d_log, float* d_radius,
                            float* d_cos, void* stream) {
    HSES_REQUIRE((uint64_t)k_lo + n <= kUnitCount, "k range exceeds 2^24");
    if (n == 0) return HSES_OK;
    DeviceState* st;
    int rc = get_state(&st);
    if (rc) return rc;
    const uint32_t blocks = std::min<uint32_t>((n + 255) / 256, 65536u);
    hipLaunchKernelGGL(k_bm_eval, dim3(blocks), dim3(256), 0, (hipStream_t)stream, k_lo, n, d_log,
                       d_radius, d_cos, st->d_tables, st->d_log_exc, st->d_cos_exc);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

static int launch_stream_rows(float bs, uint64_t key, int32_t L, int32_t epoch, int32_t nreuse,
                              int32_t tid_lo, const int32_t* tids, int32_t n, int32_t a,
                              int32_t b, float* A, float* B, void* stream,
                              const float* base = nullptr) {
    DeviceState* st;
    int rc = get_state(&st);
    if (rc) return rc;
    const uint64_t* jump;
    rc = get_jump_table(st, L, (int64_t)a + b, &jump);
    if (rc) return rc;
    const int32_t bpm = (a + b + 255) / 256;
    const int64_t blocks = (int64_t)bpm * n;
    HSES_REQUIRE(blocks < (1ll << 31), "too many members x rows");
    hipLaunchKernelGGL(k_stream_rows, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream,
                       bs, key, L, epoch, nreuse, tid_lo, tids, n, a, b, bpm, A, B, st->d_tables,
                       st->d_log_exc, st->d_cos_exc, jump, base);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

// Rows of Lc normals for a dense (a, b) block: the largest divisor of b that
// the jump tables cover (the block is one stream of a * b normals).
static int32_t dense_row_len(int32_t b) {
    int32_t Lc = std::min<int32_t>(b, kJumpMaxL);
    while (b % Lc) --Lc;
    return Lc;
}

extern "C" int hses_lora_factors(float base_sigma, uint64_t key, int32_t rank, int32_t epoch,
                                 int32_t noise_reuse, int32_t tid_lo, const int32_t* d_tids,
                                 int32_t n, int32_t a, int32_t b, float* d_A, float* d_B,
                                 void* stream) {
    HSES_REQUIRE(n >= 0 && a >= 0 && b >= 0 && rank >= 0, "negative size");
    HSES_REQUIRE(noise_reuse >= 0, "noise_reuse must be >= 0");
    if (n == 0 || rank == 0 || a + b == 0) return HSES_OK;
    HSES_REQUIRE((a == 0 || d_A) && (b == 0 || d_B), "output pointer is NULL");
    HSES_REQUIRE(d_tids || (int64_t)tid_lo + n - 1 <= INT32_MAX, "thread id overflow");
    return launch_stream_rows(base_sigma, key, rank, epoch, noise_reuse, tid_lo, d_tids, n, a, b,
                              d_A, d_B, stream);
}

extern "C" int hses_nonlora_noise(float base_sigma, uint64_t key, int32_t epoch,
                                  int32_t noise_reuse, int32_t tid_lo, const int32_t* d_tids,
                                  int32_t n, int32_t a, int32_t b, float* d_out, void* stream) {
    HSES_REQUIRE(n >= 0 && a >= 0 && b >= 0, "negative size");
    HSES_REQUIRE(noise_reuse >= 0, "noise_reuse must be >= 0");
    if (n == 0 || a == 0 || b == 0) return HSES_OK;
    HSES_REQUIRE(d_out, "output pointer is NULL");
    HSES_REQUIRE((int64_t)a * b < (1ll << 31), "a * b too large");
    // A dense (a, b) block is an A-only stream of a * b normals, written as
    // rows of Lc normals (the largest divisor of b the jump tables cover).
    const int32_t Lc = dense_row_len(b);
    return launch_stream_rows(base_sigma, key, Lc, epoch, noise_reuse, tid_lo, d_tids, n,
                              (int32_t)((int64_t)a * (b / Lc)), 0, d_out, nullptr, stream);
}

extern "C" int hses_noisy_standard(const float* d_param, int32_t a, int32_t b, uint64_t key,
                                   float sigma, int32_t epoch, int32_t noise_reuse, int32_t tid_lo,
                                   const int32_t* d_tids, int32_t n, float* d_out, void* stream) {
    HSES_REQUIRE(n >= 0 && a >= 0 && b >= 0, "negative size");
    HSES_REQUIRE(noise_reuse >= 0, "noise_reuse must be >= 0");
    if (n == 0 || a == 0 || b == 0) return HSES_OK;
    HSES_REQUIRE(d_param && d_out, "NULL pointer");
    HSES_REQUIRE((int64_t)a * b < (1ll << 31), "a * b too large");
    HSES_REQUIRE(d_tids || (int64_t)tid_lo + n - 1 <= INT32_MAX, "thread id overflow");
    const int32_t Lc = dense_row_len(b);
    return launch_stream_rows(sigma, key, Lc, epoch, noise_reuse, tid_lo, d_tids, n,
                              (int32_t)((int64_t)a * (b / Lc)), 0, d_out, nullptr, stream, d_param);
}

extern "C" size_t hses_full_update_workspace(int32_t a, int32_t b, int32_t n) {
    if (a <= 0 || b <= 0 || n <= 0) return 0;
    const int64_t E = (int64_t)a * b;
    const int32_t chunks = (int32_t)std::min<int64_t>((E + kFullLc - 1) / kFullLc, INT32_MAX);
    return (size_t)full_splits(chunks, n / 2 + 1) * (size_t)E * sizeof(double);
}

extern "C" int hses_full_update(const float* d_f, int32_t n, int32_t tid_lo, uint64_t key,
                                float sigma, int32_t epoch, int32_t noise_reuse, int32_t a,
                                int32_t b, float scale, int32_t accumulate, float* d_grad,
                                void* d_work, size_t work_bytes, void* stream) {
    HSES_REQUIRE(n >= 0 && a >= 1 && b >= 1, "bad sizes");
    HSES_REQUIRE(noise_reuse >= 0, "noise_reuse must be >= 0");
    HSES_REQUIRE(tid_lo >= 0 && (int64_t)tid_lo + n - 1 <= INT32_MAX, "thread id range");
    HSES_REQUIRE(d_grad, "grad is NULL");
    const int64_t E = (int64_t)a * b;
    const int64_t chunks = (E + kFullLc - 1) / kFullLc;
    HSES_REQUIRE(chunks <= kJumpMaxRows, "a * b exceeds 32 * 16384 elements");
    const int32_t pair_lo = tid_lo / 2, n_pairs = n ? (tid_lo + n - 1) / 2 - pair_lo + 1 : 0;
    const int32_t splits = full_splits((int32_t)chunks, n_pairs);
    const bool empty = n == 0 || sigma == 0.0f;
    if (!empty) {
        HSES_REQUIRE(d_f, "fitness is NULL");
        HSES_REQUIRE(d_work && work_bytes >= (size_t)splits * E * sizeof(double),
                     "workspace too small");
    }
    DeviceState* st;
    int rc = get_state(&st);
    if (rc) return rc;
    hipStream_t s = (hipStream_t)stream;
    const uint32_t rblocks = (uint32_t)((E + 255) / 256);
    if (empty) {
        if (!accumulate) {
            // zero gradient: reduce over no partials
            hipLaunchKernelGGL(k_full_reduce, dim3(rblocks), dim3(256), 0, s, nullptr, 0, E, scale,
                               0, d_grad);
            HSES_CHECK_HIP(hipGetLastError());
        }
        return HSES_OK;
    }
    const uint64_t* jump;
    rc = get_jump_table(st, kFullLc, chunks, &jump);
    if (rc) return rc;
    double* part = static_cast<double*>(d_work);
    hipLaunchKernelGGL(k_full_partial, dim3((uint32_t)((chunks + kFullThreads - 1) / kFullThreads),
                                            (uint32_t)splits),
                       dim3(kFullThreads), 0, s, d_f, n, tid_lo, key, sigma, epoch, noise_reuse, E,
                       (int32_t)chunks, pair_lo, n_pairs, splits, part, st->d_tables,
                       st->d_log_exc, st->d_cos_exc, jump);
    HSES_CHECK_HIP(hipGetLastError());
    hipLaunchKernelGGL(k_full_reduce, dim3(rblocks), dim3(256), 0, s, part, splits, E, scale,
                       accumulate, d_grad);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}
