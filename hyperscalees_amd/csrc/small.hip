// small.hip -- fitness, fitness normalisation, the K-chunk affine combination and
// the optimizer step.
#include <math.h>

#include "runtime.h"

namespace hses {

// snn_mnist.rs:180-201 per row, averaged over the member's rows.  Loglik:
// log_softmax(row)[label]; Binary: 1 when the first maximal class is the label.
// One wave per member, lane s taking rows s, s + 64, ...; the row values are
// summed in double (exact for these magnitudes, so the tree order of the
// cross-lane sum does not change the result).  `correct` (optional) counts
// the rows whose first maximal class is the label.
__global__ __launch_bounds__(256) void k_member_fitness(const float* __restrict__ logits,
                                                        int32_t classes,
                                                        const int32_t* __restrict__ labels,
                                                        int32_t n, int32_t rpm, int32_t reward,
                                                        float* __restrict__ fit,
                                                        unsigned long long* __restrict__ correct) {
    __shared__ uint32_t block_hits[4];
    const int32_t m = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int32_t lane = threadIdx.x & 63;
    double acc = 0.0;
    uint32_t hits = 0;
    for (int32_t s = lane; m < n && s < rpm; s += 64) {
        const int64_t row = (int64_t)m * rpm + s;
        const float* x = logits + row * classes;
        const int32_t label = labels[row];
        float mx = x[0];
        int32_t am = 0;
        for (int32_t c = 1; c < classes; ++c)
            if (x[c] > mx) {
                mx = x[c];
                am = c;
            }
        hits += am == label ? 1u : 0u;
        if (reward == HSES_REWARD_BINARY) {
            acc += am == label ? 1.0 : 0.0;
        } else {
            float sum = 0.0f;
            for (int32_t c = 0; c < classes; ++c) sum = __fadd_rn(sum, expf(__fsub_rn(x[c], mx)));
            const int32_t lab = label < 0 ? 0 : (label >= classes ? classes - 1 : label);
            acc += (double)__fsub_rn(__fsub_rn(x[lab], mx), logf(sum));
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        acc += __shfl_xor(acc, off);
        hits += __shfl_xor(hits, off);
    }
    if (lane == 0) {
        if (m < n) fit[m] = (float)(acc / rpm);
        block_hits[threadIdx.x >> 6] = hits;
    }
    if (!correct) return;  // uniform over the block
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t h = block_hits[0] + block_hits[1] + block_hits[2] + block_hits[3];
        if (h) atomicAdd(correct, (unsigned long long)h);
    }
}

// The same fitness for wide rows (classes > 64, e.g. a language model's
// vocabulary): one wave per member walks its rows in order, the lanes split a
// row's classes (coalesced loads); the row's maximum and first maximal class,
// and its sum of exponentials, are fixed-order wave reductions, and lane 0
// accumulates the member's rows in double in row order.
__global__ __launch_bounds__(256) void k_member_fitness_wide(const float* __restrict__ logits,
                                                             int32_t classes,
                                                             const int32_t* __restrict__ labels,
                                                             int32_t n, int32_t rpm, int32_t reward,
                                                             float* __restrict__ fit,
                                                             unsigned long long* __restrict__ correct) {
    __shared__ uint32_t block_hits[4];
    const int32_t m = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int32_t lane = threadIdx.x & 63;
    double acc = 0.0;
    uint32_t hits = 0;
    for (int32_t s = 0; m < n && s < rpm; ++s) {
        const int64_t row = (int64_t)m * rpm + s;
        const float* x = logits + row * classes;
        float mx = -INFINITY;
        int32_t am = classes;
        for (int32_t c = lane; c < classes; c += 64)
            if (x[c] > mx) {  // ascending c: the lane's first maximal class
                mx = x[c];
                am = c;
            }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float om = __shfl_xor(mx, off);
            const int32_t oa = __shfl_xor(am, off);
            if (om > mx || (om == mx && oa < am)) {
                mx = om;
                am = oa;
            }
        }
        const int32_t label = labels[row];
        hits += am == label ? 1u : 0u;
        if (reward == HSES_REWARD_BINARY) {
            acc += am == label ? 1.0 : 0.0;
        } else {
            float sum = 0.0f;
            for (int32_t c = lane; c < classes; c += 64) sum = __fadd_rn(sum, expf(__fsub_rn(x[c], mx)));
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) sum = __fadd_rn(sum, __shfl_xor(sum, off));
            const int32_t lab = label < 0 ? 0 : (label >= classes ? classes - 1 : label);
            acc += (double)__fsub_rn(__fsub_rn(x[lab], mx), logf(sum));
        }
    }
    if (lane == 0) {
        if (m < n) fit[m] = (float)(acc / rpm);
        block_hits[threadIdx.x >> 6] = hits;
    }
    if (!correct) return;  // uniform over the block
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t h = block_hits[0] + block_hits[1] + block_hits[2] + block_hits[3];
        if (h) atomicAdd(correct, (unsigned long long)h);
    }
}

// Sum and sum of squares (in double) of v[0..n) over one 1024-thread block,
// a fixed-order tree, so the result is deterministic.  Every thread returns
// the totals.
__device__ void block_moments(const float* __restrict__ v, int32_t n, double* s1, double* s2,
                              double& a_out, double& b_out) {
    double a = 0.0, b = 0.0;
    for (int32_t i = threadIdx.x; i < n; i += blockDim.x) {
        const float x = v[i];
        a += (double)x;
        b += (double)__fmul_rn(x, x);
    }
    s1[threadIdx.x] = a;
    s2[threadIdx.x] = b;
    __syncthreads();
    for (int32_t w = blockDim.x / 2; w > 0; w >>= 1) {
        if ((int32_t)threadIdx.x < w) {
            s1[threadIdx.x] += s1[threadIdx.x + w];
            s2[threadIdx.x] += s2[threadIdx.x + w];
        }
        __syncthreads();
    }
    a_out = s1[0];
    b_out = s2[0];
}

// eggroll.rs:967-992: mean and E[x^2] over all n (double partial sums with a
// fixed-order tree, one block), std = sqrt(var + 1e-5), out = (raw-mean)/std
// or per-group centring with the global std.
__global__ __launch_bounds__(1024) void k_convert_fitnesses(const float* __restrict__ raw,
                                                           int32_t n, int32_t group,
                                                           float* __restrict__ out,
                                                           float* __restrict__ stats) {
    __shared__ double s1[1024], s2[1024];
    double t1, t2;
    block_moments(raw, n, s1, s2, t1, t2);
    const float mean = (float)(t1 / n);
    const float msq = (float)(t2 / n);
    const float var = __fsub_rn(msq, __fmul_rn(mean, mean));
    const float sd = __fsqrt_rn(__fadd_rn(var, 1e-5f));
    const float inv = __fdiv_rn(1.0f, sd);
    if (threadIdx.x == 0 && stats) {
        stats[0] = mean;
        stats[1] = sd;
    }
    if (group <= 0) {
        for (int32_t i = threadIdx.x; i < n; i += blockDim.x)
            out[i] = __fmul_rn(__fadd_rn(raw[i], -mean), inv);
    } else {
        const int32_t groups = n / group;
        for (int32_t gi = threadIdx.x; gi < groups; gi += blockDim.x) {
            double gs = 0.0;
            for (int32_t j = 0; j < group; ++j) gs += (double)raw[gi * group + j];
            const float gm = (float)(gs / group);
            for (int32_t j = 0; j < group; ++j)
                out[gi * group + j] = __fmul_rn(__fsub_rn(raw[gi * group + j], gm), inv);
        }
    }
}

// accumulate_train.rs:843-846: the raw-fitness sums of one chunk added to
// (or, first chunk, written into) moments = {sum raw, sum raw^2}.
__global__ __launch_bounds__(1024) void k_fitness_moments(const float* __restrict__ raw, int32_t n,
                                                         double* __restrict__ moments,
                                                         int32_t accumulate) {
    __shared__ double s1[1024], s2[1024];
    double t1, t2;
    block_moments(raw, n, s1, s2, t1, t2);
    if (threadIdx.x == 0) {
        moments[0] = accumulate ? moments[0] + t1 : t1;
        moments[1] = accumulate ? moments[1] + t2 : t2;
    }
}

// combine_affine_grads (eggroll.rs:902-915) with the driver's mean and std
// (accumulate_train.rs:940-944) taken from the device moments:
// out = (g - o*mean) * (-1 / (std * sqrt(batch))).
__global__ void k_combine_affine(const float* __restrict__ g, const float* __restrict__ o,
                                 const double* __restrict__ moments, int32_t batch, int64_t len,
                                 float* __restrict__ out) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= len) return;
    const float fb = (float)batch;
    const float mean = __fdiv_rn((float)moments[0], fb);
    const float var = fmaxf(__fsub_rn(__fdiv_rn((float)moments[1], fb), __fmul_rn(mean, mean)), 0.0f);
    const float sd = __fsqrt_rn(__fadd_rn(var, 1e-5f));
    const float scale = __fdiv_rn(-1.0f, __fmul_rn(sd, __fsqrt_rn(fb)));
    const float gv = g[e];
    out[e] = __fmul_rn(o ? __fsub_rn(gv, __fmul_rn(o[e], mean)) : gv, scale);
}

// noiser.rs:155-225.  kind 0: p - g*lr.  Adam/AdamW: moments, bias correction
// (inverse factors precomputed on the host), p + (m_hat/(sqrt(v_hat)+eps))*(-lr)
// (+ p*wd for AdamW, no lr factor, as the reference).
// With gscale (TrustRegion, noiser.rs:215-222) the gradient is first
// multiplied by the clip factor *gscale, as clip_grads_global_norm does.
__global__ void k_solver(int32_t kind, float lr, float b1, float omb1, float b2, float omb2,
                         float eps, float wd, float i1, float i2, float* __restrict__ p,
                         const float* __restrict__ g, float* __restrict__ m, float* __restrict__ v,
                         int64_t len, const float* __restrict__ gscale) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= len) return;
    const float pv = p[e], gv = gscale ? __fmul_rn(g[e], gscale[0]) : g[e];
    if (kind == HSES_SGD) {
        p[e] = __fsub_rn(pv, __fmul_rn(gv, lr));
        return;
    }
    const float mn = __fadd_rn(__fmul_rn(m[e], b1), __fmul_rn(gv, omb1));
    const float vn = __fadd_rn(__fmul_rn(v[e], b2), __fmul_rn(__fmul_rn(gv, gv), omb2));
    m[e] = mn;
    v[e] = vn;
    const float mh = __fmul_rn(mn, i1), vh = __fmul_rn(vn, i2);
    const float denom = __fadd_rn(__fsqrt_rn(vh), eps);
    const float at = __fmul_rn(__fdiv_rn(mh, denom), -lr);
    p[e] = (kind == HSES_ADAMW && wd != 0.0f) ? __fadd_rn(__fadd_rn(pv, at), __fmul_rn(pv, wd))
                                               : __fadd_rn(pv, at);
}

// clip_grads_global_norm (noiser.rs:231-244), stage 1: kClipBlocks partial
// sums of g*g (the f32 square, accumulated in double) over a fixed partition
// of one tensor; each block sums its range with a fixed stride and a fixed
// tree, so the result depends on the length only.
constexpr int kClipBlocks = 64;
__global__ __launch_bounds__(256) void k_sq_partial(const float* __restrict__ g, int64_t len,
                                                    double* __restrict__ part) {
    __shared__ double red[256];
    const int64_t per = (len + kClipBlocks - 1) / kClipBlocks;
    const int64_t lo = (int64_t)blockIdx.x * per, hi = min(len, lo + per);
    double s = 0.0;
    for (int64_t e = lo + threadIdx.x; e < hi; e += 256) {
        const float v = g[e];
        s += (double)__fmul_rn(v, v);
    }
    red[threadIdx.x] = s;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) part[blockIdx.x] = red[0];
}

// Stage 2: per tensor the partials in order (double, then f32 as the
// reference's per-tensor sum), the tensors' sums added in f32 in order, and
// scale = max_norm / ||g|| when ||g|| > max_norm and ||g|| > 0, else 1.
__global__ void k_clip_scale(const double* __restrict__ part, int32_t n, float max_norm,
                             float* __restrict__ scale) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    float sq = 0.0f;
    for (int32_t i = 0; i < n; ++i) {
        double s = 0.0;
        for (int b = 0; b < kClipBlocks; ++b) s += part[(int64_t)i * kClipBlocks + b];
        sq = __fadd_rn(sq, (float)s);
    }
    const float gn = __fsqrt_rn(sq);
    scale[0] = (gn > max_norm && gn > 0.0f) ? __fdiv_rn(max_norm, gn) : 1.0f;
}

}  // namespace hses

using namespace hses;

extern "C" int hses_clip_global_norm(const float* const* h_grads, const int64_t* h_lens,
                                     int32_t n, float max_norm, double* d_work, float* d_scale,
                                     void* stream) {
    HSES_REQUIRE(n >= 1 && h_grads && h_lens, "need at least one gradient tensor");
    HSES_REQUIRE(max_norm >= 0.0f, "max_norm must be >= 0");
    HSES_REQUIRE(d_work && d_scale, "NULL pointer");
    for (int32_t i = 0; i < n; ++i) {
        HSES_REQUIRE(h_lens[i] >= 0, "negative length");
        HSES_REQUIRE(h_lens[i] == 0 || h_grads[i], "NULL gradient");
    }
    hipStream_t s = (hipStream_t)stream;
    for (int32_t i = 0; i < n; ++i) {
        hipLaunchKernelGGL(k_sq_partial, dim3(kClipBlocks), dim3(256), 0, s, h_grads[i], h_lens[i],
                           d_work + (int64_t)i * kClipBlocks);
        HSES_CHECK_HIP(hipGetLastError());
    }
    hipLaunchKernelGGL(k_clip_scale, dim3(1), dim3(64), 0, s, d_work, n, max_norm, d_scale);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_member_fitness(const float* d_logits, int32_t classes, const int32_t* d_labels,
                                   int32_t n, int32_t rows_per_member, int32_t reward, float* d_fit,
                                   unsigned long long* d_correct, void* stream) {
    HSES_REQUIRE(n >= 0 && classes >= 1 && rows_per_member >= 1, "bad sizes");
    HSES_REQUIRE(reward == HSES_REWARD_LOGLIK || reward == HSES_REWARD_BINARY, "unknown reward");
    if (n == 0) return HSES_OK;
    HSES_REQUIRE(d_logits && d_labels && d_fit, "NULL pointer");
    hipLaunchKernelGGL(classes > 64 ? k_member_fitness_wide : k_member_fitness, dim3((n + 3) / 4),
                       dim3(256), 0, (hipStream_t)stream,
                       d_logits, classes, d_labels, n, rows_per_member, reward, d_fit, d_correct);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_member_loglik(const float* d_logits, int32_t classes, const int32_t* d_labels,
                                  int32_t n, int32_t rows_per_member, float* d_fit, void* stream) {
    return hses_member_fitness(d_logits, classes, d_labels, n, rows_per_member, HSES_REWARD_LOGLIK,
                               d_fit, nullptr, stream);
}

extern "C" int hses_fitness_moments(const float* d_raw, int32_t n, double* d_moments,
                                    int32_t accumulate, void* stream) {
    HSES_REQUIRE(n >= 0, "negative n");
    HSES_REQUIRE(d_moments && (n == 0 || d_raw), "NULL pointer");
    hipLaunchKernelGGL(k_fitness_moments, dim3(1), dim3(1024), 0, (hipStream_t)stream, d_raw, n,
                       d_moments, accumulate);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_combine_affine(const float* d_grad_acc, const float* d_ones_acc,
                                   const double* d_moments, int32_t batch, int64_t len, float* d_out,
                                   void* stream) {
    HSES_REQUIRE(batch >= 1, "batch must be >= 1");
    HSES_REQUIRE(len >= 0, "negative length");
    if (len == 0) return HSES_OK;
    HSES_REQUIRE(d_grad_acc && d_moments && d_out, "NULL pointer");
    const int64_t blocks = (len + 255) / 256;
    HSES_REQUIRE(blocks < (1ll << 31), "grid too large");
    hipLaunchKernelGGL(k_combine_affine, dim3(blocks), dim3(256), 0, (hipStream_t)stream, d_grad_acc,
                       d_ones_acc, d_moments, batch, len, d_out);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_convert_fitnesses(const float* d_raw, int32_t n, int32_t group_size,
                                      float* d_out, float* d_stats, void* stream) {
    HSES_REQUIRE(n >= 1, "n must be >= 1");
    HSES_REQUIRE(d_raw && d_out, "NULL pointer");
    HSES_REQUIRE(group_size >= 0, "group_size must be >= 0");
    HSES_REQUIRE(group_size == 0 || n % group_size == 0, "n must be a multiple of group_size");
    hipLaunchKernelGGL(k_convert_fitnesses, dim3(1), dim3(1024), 0, (hipStream_t)stream, d_raw, n,
                       group_size, d_out, d_stats);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_solver_step_scaled(int32_t kind, float lr, float beta1, float beta2,
                                       float eps, float wd, int32_t step_t, float* d_param,
                                       const float* d_grad, float* d_m, float* d_v, int64_t len,
                                       const float* d_gscale, void* stream) {
    HSES_REQUIRE(kind >= HSES_SGD && kind <= HSES_ADAMW, "unknown solver");
    HSES_REQUIRE(len >= 0, "negative length");
    if (len == 0) return HSES_OK;
    HSES_REQUIRE(d_param && d_grad, "NULL pointer");
    float i1 = 1.0f, i2 = 1.0f;
    if (kind != HSES_SGD) {
        HSES_REQUIRE(d_m && d_v, "Adam moments are NULL");
        HSES_REQUIRE(step_t >= 1, "step_t must be >= 1 for Adam");
        const float t = (float)step_t;
        i1 = 1.0f / (1.0f - powf(beta1, t));
        i2 = 1.0f / (1.0f - powf(beta2, t));
    }
    const int64_t blocks = (len + 255) / 256;
    HSES_REQUIRE(blocks < (1ll << 31), "grid too large");
    hipLaunchKernelGGL(k_solver, dim3(blocks), dim3(256), 0, (hipStream_t)stream, kind, lr, beta1,
                       1.0f - beta1, beta2, 1.0f - beta2, eps, wd, i1, i2, d_param, d_grad, d_m,
                       d_v, len, d_gscale);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_solver_step(int32_t kind, float lr, float beta1, float beta2, float eps,
                                float wd, int32_t step_t, float* d_param, const float* d_grad,
                                float* d_m, float* d_v, int64_t len, void* stream) {
    return hses_solver_step_scaled(kind, lr, beta1, beta2, eps, wd, step_t, d_param, d_grad, d_m,
                                   d_v, len, nullptr, stream);
}
