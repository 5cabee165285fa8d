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
// b == 0 and A == nullptr it writes a dense (a, L) noise block instead
// (get_nonlora_update_params: all rows scaled).
__global__ __launch_bounds__(256) void k_stream_rows(float bs, uint64_t key, int32_t L, int32_t epoch, int32_t nreuse,
                              int32_t tid_lo, const int32_t* tids, int32_t n, int32_t a, int32_t b,
                              int32_t blocks_per_member, float* A, float* B,
                              const BmTables* gt, const uint32_t* le, const uint32_t* ce,
                              const uint64_t* jump) {
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
    } else {
        const float sc = sign * bs;
        float* dst = A + ((int64_t)m * a + (j - b)) * L;
        bm_run(s, L, ctx, [&](int32_t c, float v) { dst[c] = v * sc; });
    }
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
                              int32_t b, float* A, float* B, void* stream) {
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
                       st->d_log_exc, st->d_cos_exc, jump);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
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
    int32_t Lc = std::min<int32_t>(b, kJumpMaxL);
    while (b % Lc) --Lc;
    return launch_stream_rows(base_sigma, key, Lc, epoch, noise_reuse, tid_lo, d_tids, n,
                              (int32_t)((int64_t)a * (b / Lc)), 0, d_out, nullptr, stream);
}
