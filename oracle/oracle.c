/*
 * oracle.c -- CPU restatement of the reference's EggRoll SNN hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  Compiled with -ffp-contract=off so
 * that no multiply-add is fused: the reference CPU backend evaluates each
 * tensor op separately.  Citations are to files under the reference root.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* Noise stream                                                              */
/* ------------------------------------------------------------------------ */

/* burn_impl/hyperscalees-noiser/src/noiser.rs:495-506.  `i32 as u64` in Rust
 * sign-extends, so the epoch/thread are widened through int64_t. */
uint64_t or_noise_seed(uint64_t key, int32_t true_epoch, int32_t true_thread) {
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

/* burn_impl/hyperscalees-noiser/src/eggroll.rs:60-65 */
void or_epoch_thread_sign(int32_t epoch, int32_t thread_id, int32_t noise_reuse,
                          int32_t *true_epoch, int32_t *true_thread, float *sign) {
    *true_epoch = noise_reuse == 0 ? 0 : epoch / noise_reuse;
    *true_thread = thread_id / 2;
    *sign = (thread_id % 2 == 0) ? 1.0f : -1.0f;
}

/* noiser.rs:453-460 (DeterministicNoise::next_u64) */
uint64_t or_xorshift64_step(uint64_t x) {
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    return x;
}

/* noiser.rs:462-466 (next_unit): 24 high bits scaled by 2^-24. */
float or_unit_from_u64(uint64_t x) { return (float)(x >> 40) / 16777216.0f; }

/* noiser.rs:470-477, radius half of standard_normal for unit index k1. */
float or_bm_radius(uint32_t k1) {
    float u1 = (float)k1 / 16777216.0f;
    u1 = u1 > 1e-9f ? u1 : 1e-9f; /* f32::max(1e-9) */
    float l = logf(u1);
    return sqrtf(-2.0f * l);
}

/* noiser.rs:475-476, angle half: cos(TAU * u2) with TAU = std::f32::consts::TAU. */
float or_bm_cos(uint32_t k2) {
    const float TAU = 6.28318530717958647692f;
    float u2 = (float)k2 / 16777216.0f;
    float theta = TAU * u2;
    return cosf(theta);
}

void or_bm_eval(uint32_t k_lo, uint32_t n, float *lg, float *rad, float *cs) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int64_t i = 0; i < (int64_t)n; ++i) {
        const uint32_t k = k_lo + (uint32_t)i;
        float u1 = (float)k / 16777216.0f;
        u1 = u1 > 1e-9f ? u1 : 1e-9f;
        const float l = logf(u1);
        if (lg) lg[i] = l;
        if (rad) rad[i] = sqrtf(-2.0f * l);
        if (cs) cs[i] = or_bm_cos(k);
    }
}

/* noiser.rs:448-490: state = seed | 1; each normal consumes two steps. */
void or_standard_normals(uint64_t seed, float *out, int64_t n) {
    uint64_t s = seed | 1ull;
    for (int64_t i = 0; i < n; ++i) {
        s = or_xorshift64_step(s);
        uint32_t k1 = (uint32_t)(s >> 40);
        s = or_xorshift64_step(s);
        uint32_t k2 = (uint32_t)(s >> 40);
        out[i] = or_bm_radius(k1) * or_bm_cos(k2);
    }
}

/* ------------------------------------------------------------------------ */
/* EggRoll factors                                                           */
/* ------------------------------------------------------------------------ */

/* eggroll.rs:433 / :365: base_sigma = sigma / (rank as f32).sqrt() */
float or_base_sigma(float sigma, int32_t rank) { return sigma / sqrtf((float)rank); }

/* eggroll.rs:86-103.  Stream of (a+b)*r normals, row-major (a+b, r):
 * rows [0,b) are B, rows [b,a+b) are A, A scaled by sign*base_sigma. */
void or_get_lora_update_params(float base_sigma, uint64_t key, int32_t rank,
                               int32_t epoch, int32_t thread_id, int32_t a, int32_t b,
                               int32_t noise_reuse, float *A, float *B) {
    int32_t te, tt;
    float sign;
    or_epoch_thread_sign(epoch, thread_id, noise_reuse, &te, &tt, &sign);
    int64_t n = (int64_t)(a + b) * rank;
    float *buf = (float *)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
    or_standard_normals(or_noise_seed(key, te, tt), buf, n);
    const float sc = sign * base_sigma;
    memcpy(B, buf, sizeof(float) * (size_t)b * (size_t)rank);
    for (int64_t i = 0; i < (int64_t)a * rank; ++i) A[i] = buf[(int64_t)b * rank + i] * sc;
    free(buf);
}

/* eggroll.rs:116-227: generate_lora_flat multiplies the A region by sign, then
 * lora_flat_to_tensors multiplies by base_sigma; IEEE sign symmetry makes that
 * identical to one multiply by sign*base_sigma, so the per-thread routine is reused. */
void or_batched_lora_noise(float base_sigma, uint64_t key, int32_t rank,
                           const int32_t *tids, int32_t n, int32_t epoch, int32_t noise_reuse,
                           int32_t a, int32_t b, float *A, float *B) {
    for (int32_t i = 0; i < n; ++i) {
        float *Ai = A + (int64_t)i * a * rank;
        float *Bi = B + (int64_t)i * b * rank;
        int32_t te, tt;
        float sign;
        or_epoch_thread_sign(epoch, tids[i], noise_reuse, &te, &tt, &sign);
        int64_t len = (int64_t)(a + b) * rank;
        float *buf = (float *)malloc(sizeof(float) * (size_t)(len > 0 ? len : 1));
        or_standard_normals(or_noise_seed(key, te, tt), buf, len);
        memcpy(Bi, buf, sizeof(float) * (size_t)b * (size_t)rank);
        for (int64_t k = 0; k < (int64_t)a * rank; ++k)
            Ai[k] = (buf[(int64_t)b * rank + k] * sign) * base_sigma;
        free(buf);
    }
}

/* eggroll.rs:312-324 */
void or_get_nonlora_update_params(float base_sigma, uint64_t key, int32_t epoch,
                                  int32_t thread_id, int32_t a, int32_t b, int32_t noise_reuse,
                                  float *out) {
    int32_t te, tt;
    float sign;
    or_epoch_thread_sign(epoch, thread_id, noise_reuse, &te, &tt, &sign);
    int64_t n = (int64_t)a * b;
    or_standard_normals(or_noise_seed(key, te, tt), out, n);
    const float sc = sign * base_sigma;
    for (int64_t i = 0; i < n; ++i) out[i] = out[i] * sc;
}

/* ------------------------------------------------------------------------ */
/* Matrix products                                                           */
/* ------------------------------------------------------------------------ */

/* y(m,n) = x(m,k) @ w(n,k)^T with f32 accumulation in ascending k.  The loop
 * runs i-k-j over a transposed copy of w so the j loop vectorises without
 * changing the per-element summation order. */
void or_matmul_abt(const float *x, int32_t m, int32_t k, const float *w, int32_t n, float *y) {
    float *wt = (float *)malloc(sizeof(float) * (size_t)k * (size_t)n + 4);
    for (int32_t j = 0; j < n; ++j)
        for (int32_t kk = 0; kk < k; ++kk) wt[(int64_t)kk * n + j] = w[(int64_t)j * k + kk];
    for (int32_t i = 0; i < m; ++i) {
        float *yi = y + (int64_t)i * n;
        for (int32_t j = 0; j < n; ++j) yi[j] = 0.0f;
        const float *xi = x + (int64_t)i * k;
        for (int32_t kk = 0; kk < k; ++kk) {
            const float xv = xi[kk];
            const float *wr = wt + (int64_t)kk * n;
            for (int32_t j = 0; j < n; ++j) yi[j] = yi[j] + xv * wr[j];
        }
    }
    free(wt);
}

void or_matmul_abt_f64(const float *x, int32_t m, int32_t k, const float *w, int32_t n,
                       float *y) {
    double *acc = (double *)malloc(sizeof(double) * (size_t)(n > 0 ? n : 1));
    for (int32_t i = 0; i < m; ++i) {
        for (int32_t j = 0; j < n; ++j) {
            double s = 0.0;
            const float *xi = x + (int64_t)i * k, *wj = w + (int64_t)j * k;
            for (int32_t kk = 0; kk < k; ++kk) s += (double)xi[kk] * (double)wj[kk];
            acc[j] = s;
        }
        for (int32_t j = 0; j < n; ++j) y[(int64_t)i * n + j] = (float)acc[j];
    }
    free(acc);
}

/* y(m,n) = x(m,k) @ w(k,n), f32 accumulation in ascending k. */
static void matmul_ab(const float *x, int32_t m, int32_t k, const float *w, int32_t n, float *y) {
    for (int32_t i = 0; i < m; ++i) {
        float *yi = y + (int64_t)i * n;
        for (int32_t j = 0; j < n; ++j) yi[j] = 0.0f;
        const float *xi = x + (int64_t)i * k;
        for (int32_t kk = 0; kk < k; ++kk) {
            const float xv = xi[kk];
            const float *wr = w + (int64_t)kk * n;
            for (int32_t j = 0; j < n; ++j) yi[j] = yi[j] + xv * wr[j];
        }
    }
}

/* eggroll.rs:419-446 (do_mm_impl): base = x@W^T; base + (x@B)@A^T. */
void or_do_mm(const float *x, int32_t rows, const float *W, int32_t a, int32_t b,
              const float *A, const float *B, int32_t r, float *y) {
    or_matmul_abt(x, rows, b, W, a, y);
    if (!A || !B) return;
    float *xb = (float *)malloc(sizeof(float) * (size_t)rows * (size_t)r + 4);
    float *z = (float *)malloc(sizeof(float) * (size_t)rows * (size_t)a + 4);
    matmul_ab(x, rows, b, B, r, xb);  /* (rows,b)@(b,r) */
    or_matmul_abt(xb, rows, r, A, a, z); /* (rows,r)@(a,r)^T */
    for (int64_t i = 0; i < (int64_t)rows * a; ++i) y[i] = y[i] + z[i];
    free(xb);
    free(z);
}

/* eggroll.rs:450-477 (do_Tmm_impl): base = x@W; base + (x@A)@B^T with W (a,b). */
void or_do_Tmm(const float *x, int32_t rows, const float *W, int32_t a, int32_t b,
               const float *A, const float *B, int32_t r, float *y) {
    matmul_ab(x, rows, a, W, b, y);
    if (!A || !B) return;
    float *xa = (float *)malloc(sizeof(float) * (size_t)rows * (size_t)r + 4);
    float *z = (float *)malloc(sizeof(float) * (size_t)rows * (size_t)b + 4);
    matmul_ab(x, rows, a, A, r, xa);
    or_matmul_abt(xa, rows, r, B, b, z);
    for (int64_t i = 0; i < (int64_t)rows * b; ++i) y[i] = y[i] + z[i];
    free(xa);
    free(z);
}

/* ------------------------------------------------------------------------ */
/* SNN pieces                                                                */
/* ------------------------------------------------------------------------ */

/* burn_impl/hyperscalees-models/src/snn.rs:53-97 (lif_step / run_lif):
 * leak = dt/tau_m; charged = v + ((-v) + c) * leak; spike = charged >= v_th;
 * v = charged * (1 - spike).  Each op rounds separately (no FMA). */
void or_lif_scan(const float *cur, const float *v0, int32_t T, int64_t M, int32_t h,
                 float tau_m, float v_th, float *spikes, float *v_out) {
    const float leak = 1.0f / tau_m;
    const int64_t plane = M * h;
    for (int64_t e = 0; e < plane; ++e) {
        float v = v0 ? v0[e] : 0.0f;
        for (int32_t t = 0; t < T; ++t) {
            const float c = cur[(int64_t)t * plane + e];
            const float d = -v + c;
            const float charged = v + d * leak;
            const float s = charged >= v_th ? 1.0f : 0.0f;
            v = charged * (-s + 1.0f);
            spikes[(int64_t)t * plane + e] = s;
        }
        if (v_out) v_out[e] = v;
    }
}

/* burn_impl/hyperscalees-kernels/src/poisson_encode_fused_oxide.rs:35-106:
 * per flat element idx, xorshift32 (13,17,5) seeded
 * 1000000007*idx + (s0^s1^s2^s3) + 0x9E3779B9; u = ((v>>9)+1)/8388609;
 * spike = u < p.  The reference unrolls T<=8; the same recurrence continues for
 * larger T. */
void or_poisson_encode(const float *p, int64_t M, int32_t in_dim, int32_t T, uint32_t s0,
                       uint32_t s1, uint32_t s2, uint32_t s3, float *spikes) {
    const int64_t total = M * in_dim;
    const uint32_t mix = s0 ^ s1 ^ s2 ^ s3;
    for (int64_t idx = 0; idx < total; ++idx) {
        uint32_t x = 1000000007u * (uint32_t)idx + mix + 0x9E3779B9u;
        const float pv = p[idx];
        for (int32_t t = 0; t < T; ++t) {
            x ^= x << 13;
            x ^= x >> 17;
            x ^= x << 5;
            const float u = ((float)(x >> 9) + 1.0f) / 8388609.0f;
            spikes[(int64_t)t * total + idx] = u < pv ? 1.0f : 0.0f;
        }
    }
}

/* snn.rs:274: spikes.mean_dim(0): sum over T (exact for 0/1) divided by T. */
void or_mean_rate(const float *spikes, int32_t T, int64_t M, int32_t h, float *rate) {
    const int64_t plane = M * h;
    for (int64_t e = 0; e < plane; ++e) {
        float s = 0.0f;
        for (int32_t t = 0; t < T; ++t) s = s + spikes[(int64_t)t * plane + e];
        rate[e] = s / (float)T;
    }
}

/* ------------------------------------------------------------------------ */
/* Fitness                                                                   */
/* ------------------------------------------------------------------------ */

/* burn_impl/hyperscalees-envs/src/snn_mnist.rs:180-201 (Reward::Loglik):
 * log_softmax(logits)[label] = (x - max)[label] - ln(sum exp(x - max)). */
void or_loglik(const float *logits, int64_t rows, int32_t classes, const int32_t *labels,
               float *out) {
    for (int64_t i = 0; i < rows; ++i) {
        const float *x = logits + i * classes;
        float mx = x[0];
        for (int32_t c = 1; c < classes; ++c) mx = x[c] > mx ? x[c] : mx;
        float s = 0.0f;
        for (int32_t c = 0; c < classes; ++c) s = s + expf(x[c] - mx);
        out[i] = (x[labels[i]] - mx) - logf(s);
    }
}

/* burn_impl/hyperscalees-noiser/src/eggroll.rs:967-992 / noiser.rs:517-537.
 * mean and E[x^2] accumulate in double (the reference's reduction order is
 * backend-defined); var = E[x^2] - mean^2; std = sqrt(var + 1e-5). */
void or_convert_fitnesses(const float *raw, int32_t n, int32_t group_size, float *out,
                          float *mean_out, float *std_out) {
    double s = 0.0, s2 = 0.0;
    for (int32_t i = 0; i < n; ++i) {
        s += raw[i];
        s2 += (double)(raw[i] * raw[i]);
    }
    const float mean = (float)(s / n);
    const float msq = (float)(s2 / n);
    const float var = msq - mean * mean;
    const float std = sqrtf(var + 1e-5f);
    const float inv = 1.0f / std;
    if (mean_out) *mean_out = mean;
    if (std_out) *std_out = std;
    if (group_size <= 0) {
        for (int32_t i = 0; i < n; ++i) out[i] = (raw[i] + (-mean)) * inv;
    } else {
        const int32_t groups = n / group_size;
        for (int32_t g = 0; g < groups; ++g) {
            double gs = 0.0;
            for (int32_t j = 0; j < group_size; ++j) gs += raw[g * group_size + j];
            const float gm = (float)(gs / group_size);
            for (int32_t j = 0; j < group_size; ++j)
                out[g * group_size + j] = (raw[g * group_size + j] - gm) * inv;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* ES update                                                                 */
/* ------------------------------------------------------------------------ */

/* eggroll.rs:353-373 (_simple_lora_update): acc += (A_i@B_i^T)*f_i in member
 * order, then * (1/N). */
void or_simple_lora_update(float sigma, uint64_t key, int32_t rank, int32_t noise_reuse,
                           const float *scores, const int32_t *epochs, const int32_t *tids,
                           int32_t n, int32_t a, int32_t b, float *g) {
    const float bs = or_base_sigma(sigma, rank);
    float *A = (float *)malloc(sizeof(float) * (size_t)a * (size_t)rank + 4);
    float *B = (float *)malloc(sizeof(float) * (size_t)b * (size_t)rank + 4);
    float *ab = (float *)malloc(sizeof(float) * (size_t)a * (size_t)b + 4);
    memset(g, 0, sizeof(float) * (size_t)a * (size_t)b);
    for (int32_t i = 0; i < n; ++i) {
        or_get_lora_update_params(bs, key, rank, epochs[i], tids[i], a, b, noise_reuse, A, B);
        or_matmul_abt(A, a, rank, B, b, ab); /* (a,r)@(b,r)^T */
        for (int64_t e = 0; e < (int64_t)a * b; ++e) g[e] = g[e] + ab[e] * scores[i];
    }
    const float invn = 1.0f / (float)n;
    for (int64_t e = 0; e < (int64_t)a * b; ++e) g[e] = g[e] * invn;
    free(A);
    free(B);
    free(ab);
}

/* eggroll.rs:384-404 (_do_update, map_class 1): -(g * sqrt(N)). */
void or_do_update_lora(float sigma, uint64_t key, int32_t rank, int32_t noise_reuse,
                       const float *scores, const int32_t *epochs, const int32_t *tids,
                       int32_t n, int32_t a, int32_t b, float *grad) {
    or_simple_lora_update(sigma, key, rank, noise_reuse, scores, epochs, tids, n, a, b, grad);
    const float sq = sqrtf((float)n);
    for (int64_t e = 0; e < (int64_t)a * b; ++e) grad[e] = -(grad[e] * sq);
}

/* eggroll.rs:331-350 + 384-404 (map_class 0, _simple_full_update). */
void or_do_update_full(float sigma, uint64_t key, int32_t noise_reuse, int32_t freeze_nonlora,
                       const float *scores, const int32_t *epochs, const int32_t *tids,
                       int32_t n, int32_t a, int32_t b, float *grad) {
    const int64_t len = (int64_t)a * b;
    memset(grad, 0, sizeof(float) * (size_t)len);
    if (!freeze_nonlora) {
        float *up = (float *)malloc(sizeof(float) * (size_t)len + 4);
        for (int32_t i = 0; i < n; ++i) {
            or_get_nonlora_update_params(sigma, key, epochs[i], tids[i], a, b, noise_reuse, up);
            for (int64_t e = 0; e < len; ++e) grad[e] = grad[e] + up[e] * scores[i];
        }
        free(up);
        const float invn = 1.0f / (float)n;
        for (int64_t e = 0; e < len; ++e) grad[e] = grad[e] * invn;
    }
    const float sq = sqrtf((float)n);
    for (int64_t e = 0; e < len; ++e) grad[e] = -(grad[e] * sq);
}

/* Double-accumulated sum_i f_i * A_i @ B_i^T (reference of the reference for
 * the GPU contraction; same factors as eggroll.rs:86-103). */
void or_lora_einsum_f64(float base_sigma, uint64_t key, int32_t rank, int32_t noise_reuse,
                        int32_t epoch, const float *scores, const int32_t *tids, int32_t n,
                        int32_t a, int32_t b, double *g) {
    float *A = (float *)malloc(sizeof(float) * (size_t)a * (size_t)rank + 4);
    float *B = (float *)malloc(sizeof(float) * (size_t)b * (size_t)rank + 4);
    memset(g, 0, sizeof(double) * (size_t)a * (size_t)b);
    for (int32_t i = 0; i < n; ++i) {
        or_get_lora_update_params(base_sigma, key, rank, epoch, tids[i], a, b, noise_reuse, A,
                                  B);
        const double f = scores[i];
        for (int32_t p = 0; p < a; ++p)
            for (int32_t c = 0; c < rank; ++c) {
                const double av = f * (double)A[(int64_t)p * rank + c];
                double *gr = g + (int64_t)p * b;
                for (int32_t q = 0; q < b; ++q) gr[q] += av * (double)B[(int64_t)q * rank + c];
            }
    }
    free(A);
    free(B);
}

/* eggroll.rs:579-702 (accumulated_update_cached, LoRA branch): per chunk,
 * einsum_k = A_w_flat^T @ B_flat over (n*r); acc += einsum_k; finally
 * acc * (-1/sqrt(chunk*accumulate)). */
void or_accumulated_lora_grad(float sigma, uint64_t key, int32_t rank, int32_t noise_reuse,
                              int32_t epoch, const float *conv_full, const int32_t *tids,
                              int32_t accumulate, int32_t chunk, int32_t a, int32_t b,
                              float *grad) {
    const float bs = or_base_sigma(sigma, rank);
    const int64_t len = (int64_t)a * b;
    float *A = (float *)malloc(sizeof(float) * (size_t)chunk * a * rank + 4);
    float *B = (float *)malloc(sizeof(float) * (size_t)chunk * b * rank + 4);
    float *gk = (float *)malloc(sizeof(float) * (size_t)len + 4);
    memset(grad, 0, sizeof(float) * (size_t)len);
    for (int32_t k = 0; k < accumulate; ++k) {
        const int32_t lo = k * chunk;
        or_batched_lora_noise(bs, key, rank, tids + lo, chunk, epoch, noise_reuse, a, b, A, B);
        /* a_w = a_t * score: (n,a,r) weighted per member. */
        for (int32_t i = 0; i < chunk; ++i)
            for (int64_t e = 0; e < (int64_t)a * rank; ++e)
                A[(int64_t)i * a * rank + e] = A[(int64_t)i * a * rank + e] * conv_full[lo + i];
        /* einsum over (n, r) in row order of the flattened (n*r) axis. */
        for (int64_t e = 0; e < len; ++e) gk[e] = 0.0f;
        for (int32_t i = 0; i < chunk; ++i)
            for (int32_t c = 0; c < rank; ++c)
                for (int32_t p = 0; p < a; ++p) {
                    const float av = A[((int64_t)i * a + p) * rank + c];
                    float *gr = gk + (int64_t)p * b;
                    for (int32_t q = 0; q < b; ++q)
                        gr[q] = gr[q] + av * B[((int64_t)i * b + q) * rank + c];
                }
        for (int64_t e = 0; e < len; ++e) grad[e] = grad[e] + gk[e];
    }
    const float scale = -1.0f / sqrtf((float)(chunk * accumulate));
    for (int64_t e = 0; e < len; ++e) grad[e] = grad[e] * scale;
    free(A);
    free(B);
    free(gk);
}

/* eggroll.rs:726-748: (n,r,a)/(n,r,b) layouts, einsum('nri,nrj->ij'). */
void or_lora_einsum_raw(const float *a_t, const float *b_t, const float *scores, int32_t n,
                        int32_t r, int32_t a, int32_t b, float *g) {
    memset(g, 0, sizeof(float) * (size_t)a * (size_t)b);
    for (int32_t i = 0; i < n; ++i)
        for (int32_t c = 0; c < r; ++c)
            for (int32_t p = 0; p < a; ++p) {
                const float av = a_t[((int64_t)i * r + c) * a + p] * scores[i];
                for (int32_t q = 0; q < b; ++q)
                    g[(int64_t)p * b + q] =
                        g[(int64_t)p * b + q] + av * b_t[((int64_t)i * r + c) * b + q];
            }
}

void or_lora_einsum_ones(const float *a_t, const float *b_t, int32_t n, int32_t r, int32_t a,
                         int32_t b, float *g) {
    memset(g, 0, sizeof(float) * (size_t)a * (size_t)b);
    for (int32_t i = 0; i < n; ++i)
        for (int32_t c = 0; c < r; ++c)
            for (int32_t p = 0; p < a; ++p) {
                const float av = a_t[((int64_t)i * r + c) * a + p];
                for (int32_t q = 0; q < b; ++q)
                    g[(int64_t)p * b + q] =
                        g[(int64_t)p * b + q] + av * b_t[((int64_t)i * r + c) * b + q];
            }
}

/* eggroll.rs:902-915 */
void or_combine_affine(const float *grad_acc, const float *ones_acc, int64_t len, float mean,
                       float std, int32_t batch, float *out) {
    const float scale = -1.0f / (std * sqrtf((float)batch));
    for (int64_t e = 0; e < len; ++e) out[e] = (grad_acc[e] - ones_acc[e] * mean) * scale;
}

/* ------------------------------------------------------------------------ */
/* Solver                                                                    */
/* ------------------------------------------------------------------------ */

/* burn_impl/hyperscalees-noiser/src/noiser.rs:155-225.  AdamW adds +wd*p with
 * no lr factor, as the reference does (noiser.rs:208-212). */
void or_solver_step(int32_t kind, float lr, float beta1, float beta2, float eps, float wd,
                    int32_t step_t, const float *p, const float *g, float *m, float *v,
                    int64_t len, float *p_out) {
    if (kind == OR_SGD) {
        for (int64_t e = 0; e < len; ++e) p_out[e] = p[e] - g[e] * lr;
        return;
    }
    const float t = (float)step_t;
    const float bc1 = 1.0f - powf(beta1, t);
    const float bc2 = 1.0f - powf(beta2, t);
    const float i1 = 1.0f / bc1, i2 = 1.0f / bc2;
    const float w = kind == OR_ADAMW ? wd : 0.0f;
    for (int64_t e = 0; e < len; ++e) {
        const float mn = m[e] * beta1 + g[e] * (1.0f - beta1);
        const float vn = v[e] * beta2 + (g[e] * g[e]) * (1.0f - beta2);
        m[e] = mn;
        v[e] = vn;
        const float mh = mn * i1, vh = vn * i2;
        const float denom = sqrtf(vh) + eps;
        const float at = (mh / denom) * (-lr);
        p_out[e] = w == 0.0f ? p[e] + at : (p[e] + at) + p[e] * w;
    }
}

/* noiser.rs:231-244 (clip_grads_global_norm): returns the scale to apply. */
float or_clip_global_norm_scale(const float *const *grads, const int64_t *lens, int32_t n,
                                float max_norm) {
    float sq = 0.0f;
    for (int32_t i = 0; i < n; ++i) {
        double s = 0.0;
        for (int64_t e = 0; e < lens[i]; ++e) s += (double)(grads[i][e] * grads[i][e]);
        sq = sq + (float)s;
    }
    const float gn = sqrtf(sq);
    return (gn > max_norm && gn > 0.0f) ? max_norm / gn : 1.0f;
}

/* ------------------------------------------------------------------------ */
/* Whole SNN-MLP forward per member                                          */
/* ------------------------------------------------------------------------ */

/* Composition of snn.rs:253-282 generalised to n_layers-1 hidden LIF layers
 * (the JAX model is depth-generic: llm_experiments/snn_mnist_train_multi_gpu.py:49-98),
 * the batched LoRA forward snn.rs:665-685 per member, the rate readout and the
 * log-likelihood fitness snn_mnist.rs:180-201 averaged over the member's rows. */
/* probs / labels are member m's own R rows; m fixes its factors and the global
 * (row, col) index of its Poisson streams. */
static void snn_member(const or_snn_cfg *cfg, const float *const *W, const uint64_t *keys,
                       const float *probs, const int32_t *labels, int32_t m, float *fit_out) {
    const int32_t L = cfg->n_layers, T = cfg->T, R = cfg->rows, r = cfg->rank;
    const int32_t in0 = cfg->dims[0];
    const float bs = or_base_sigma(cfg->sigma, r);
    int32_t maxw = 0;
    for (int32_t l = 0; l <= L; ++l) maxw = cfg->dims[l] > maxw ? cfg->dims[l] : maxw;
    /* Poisson spikes for this member's rows.  The flat element index is the
     * global (row, col) index so the result equals a full-population encode. */
    float *x = (float *)malloc(sizeof(float) * (size_t)T * R * maxw + 4);
    float *y = (float *)malloc(sizeof(float) * (size_t)T * R * maxw + 4);
    const uint32_t mix =
        cfg->poisson_seed[0] ^ cfg->poisson_seed[1] ^ cfg->poisson_seed[2] ^ cfg->poisson_seed[3];
    for (int32_t s = 0; s < R; ++s)
        for (int32_t c = 0; c < in0; ++c) {
            const int64_t idx = ((int64_t)m * R + s) * in0 + c;
            uint32_t xs = 1000000007u * (uint32_t)idx + mix + 0x9E3779B9u;
            const float pv = probs[(int64_t)s * in0 + c];
            for (int32_t t = 0; t < T; ++t) {
                xs ^= xs << 13;
                xs ^= xs >> 17;
                xs ^= xs << 5;
                const float u = ((float)(xs >> 9) + 1.0f) / 8388609.0f;
                x[((int64_t)t * R + s) * in0 + c] = u < pv ? 1.0f : 0.0f;
            }
        }
    int32_t rows_cur = T * R; /* hidden layers see all (t, s) rows */
    for (int32_t l = 0; l < L; ++l) {
        const int32_t b = cfg->dims[l], a = cfg->dims[l + 1];
        float *A = (float *)malloc(sizeof(float) * (size_t)a * r + 4);
        float *B = (float *)malloc(sizeof(float) * (size_t)b * r + 4);
        or_get_lora_update_params(bs, keys[l], r, cfg->epoch, m, a, b, cfg->noise_reuse, A, B);
        if (l == L - 1) {
            /* readout on mean rates (snn.rs:274-280) */
            float *rate = (float *)malloc(sizeof(float) * (size_t)R * b + 4);
            or_mean_rate(x, T, R, b, rate);
            or_do_mm(rate, R, W[l], a, b, A, B, r, y);
            float *ll = (float *)malloc(sizeof(float) * (size_t)R + 4);
            or_loglik(y, R, a, labels, ll);
            double s = 0.0;
            for (int32_t i = 0; i < R; ++i) s += ll[i];
            *fit_out = (float)(s / R);
            free(ll);
            free(rate);
        } else {
            or_do_mm(x, rows_cur, W[l], a, b, A, B, r, y); /* (T*R, a) currents */
            or_lif_scan(y, NULL, T, R, a, cfg->tau_m, cfg->v_th, x, NULL);
        }
        free(A);
        free(B);
    }
    free(x);
    free(y);
}

void or_snn_forward_members(const or_snn_cfg *cfg, const float *const *W, const uint64_t *keys,
                            const float *probs, const int32_t *labels, int32_t m_lo,
                            int32_t m_hi, int32_t nthreads, float *fit) {
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads > 0 ? nthreads : 1)
#endif
    for (int32_t m = m_lo; m < m_hi; ++m)
        snn_member(cfg, W, keys, probs + (int64_t)m * cfg->rows * cfg->dims[0],
                   labels + (int64_t)m * cfg->rows, m, &fit[m - m_lo]);
    (void)nthreads;
}

void or_snn_forward_member(const or_snn_cfg *cfg, const float *const *W, const uint64_t *keys,
                           const float *probs_m, const int32_t *labels_m, int32_t m, float *fit) {
    snn_member(cfg, W, keys, probs_m, labels_m, m, fit);
}

void or_lora_grad_f64(float sigma, uint64_t key, int32_t rank, int32_t noise_reuse,
                      int32_t epoch, const float *fit, int32_t n, int32_t a, int32_t b,
                      int32_t nthreads, float *grad) {
    const float bs = or_base_sigma(sigma, rank);
    const int64_t len = (int64_t)a * b;
    int32_t nt = nthreads > 0 ? nthreads : 1;
    double *part = (double *)calloc((size_t)nt * (size_t)len, sizeof(double));
#ifdef _OPENMP
#pragma omp parallel num_threads(nt)
#endif
    {
        int32_t tid = 0;
#ifdef _OPENMP
        tid = omp_get_thread_num();
#endif
        double *g = part + (int64_t)tid * len;
        float *A = (float *)malloc(sizeof(float) * (size_t)a * rank + 4);
        float *B = (float *)malloc(sizeof(float) * (size_t)b * rank + 4);
        for (int32_t i = tid; i < n; i += nt) {
            or_get_lora_update_params(bs, key, rank, epoch, i, a, b, noise_reuse, A, B);
            const double f = fit[i];
            for (int32_t p = 0; p < a; ++p)
                for (int32_t c = 0; c < rank; ++c) {
                    const double av = f * (double)A[(int64_t)p * rank + c];
                    double *gr = g + (int64_t)p * b;
                    for (int32_t q = 0; q < b; ++q) gr[q] += av * (double)B[(int64_t)q * rank + c];
                }
        }
        free(A);
        free(B);
    }
    const double scale = -sqrt((double)n) / (double)n;
    for (int64_t e = 0; e < len; ++e) {
        double s = 0.0;
        for (int32_t t = 0; t < nt; ++t) s += part[(int64_t)t * len + e];
        grad[e] = (float)(s * scale);
    }
    free(part);
}
