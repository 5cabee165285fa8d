// attention.hip -- the spiking self-attention transformer's own kernels (C4).
//
// Model: src/hyperscalees/models/snn_self_attention_heads.py (LIF-encoded
// Q/K/V, multi-head attention whose row weights come from a LIF competition,
// row_softmax_lif of snn_self_attention.py:45-80, a LIF-gated feed-forward
// and a pooled readout).  The perturbed projections run on the forward
// kernels of linear*.hip; these kernels cover what lies between them, batched
// over the population: member m owns rows [m R, (m+1) R) of every (rows, C)
// plane (R = tokens per member).  Thresholds, beta and gains are per-member
// device arrays (the member's perturbed Parameter leaves after softplus).
// All arithmetic is f32 in the reference's operation order; reductions of
// spike counts are exact (integers), the attention dot products and A @ V
// sum in index order.
#include "runtime.h"

namespace hses {

namespace {

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}

// Reduction over the 64 lanes of a wave, the result in every lane: within
// rows of 16 lanes by DPP (quad swaps, then the half-row and row mirrors),
// across rows by the permlane16 and permlane32 swaps (no LDS round trips).
// Callers reduce values whose result does not depend on the order (integer
// counts, maxima).
template <class Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
    v = op(v, dpp_mov<0xB1>(v));   // quad_perm 1,0,3,2
    v = op(v, dpp_mov<0x4E>(v));   // quad_perm 2,3,0,1
    v = op(v, dpp_mov<0x141>(v));  // row_half_mirror
    v = op(v, dpp_mov<0x140>(v));  // row_mirror
    const uint32_t u = __float_as_uint(v);
    const auto p16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    v = op(__uint_as_float(p16[0]), __uint_as_float(p16[1]));
    const uint32_t w = __float_as_uint(v);
    const auto p32 = __builtin_amdgcn_permlane32_swap(w, w, false, false);
    return op(__uint_as_float(p32[0]), __uint_as_float(p32[1]));
}

__device__ __forceinline__ float wsum(float v) {
    return wave_reduce(v, [](float x, float y) { return x + y; });
}

__device__ __forceinline__ float wmax(float v) {
    return wave_reduce(v, [](float x, float y) { return fmaxf(x, y); });
}

// snn_attention.py:41-49 (dt = 1): v + leak * (-v + cur); spike = v >= vth;
// v * (1 - spike).
__device__ __forceinline__ float lif_upd(float v, float cur, float leak, float vth, float* s) {
    const float vn = __fadd_rn(v, __fmul_rn(leak, __fadd_rn(-v, cur)));
    const float sp = vn >= vth ? 1.0f : 0.0f;
    *s = sp;
    return __fmul_rn(vn, __fsub_rn(1.0f, sp));
}

}  // namespace

// jax.nn.softplus = logaddexp(x, 0) = max(x, 0) + log1p(exp(-|x|)).
__global__ __launch_bounds__(256) void k_softplus(const float* __restrict__ x, int64_t n,
                                                  float* __restrict__ y) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e < n) {
        const float v = x[e];
        y[e] = __fadd_rn(fmaxf(v, 0.0f), log1pf(expf(-fabsf(v))));
    }
}

// _rate of the three encoders and their mean plus the position embedding
// (snn_self_attention_heads.py:33-40, 168-175): one thread per (row, column).
// th_q, th_k, th_v: (n) thresholds; pos: (R, d) shared or (n, R, d).
__global__ __launch_bounds__(256) void k_sa_encode(const float* __restrict__ cq,
                                                   const float* __restrict__ ck,
                                                   const float* __restrict__ cv, int32_t T,
                                                   int64_t M, int32_t d, int32_t R,
                                                   const float* __restrict__ th_q,
                                                   const float* __restrict__ th_k,
                                                   const float* __restrict__ th_v, float leak,
                                                   const float* __restrict__ pos,
                                                   int32_t pos_per_member, float* __restrict__ X) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t total = M * d;
    if (e >= total) return;
    const int64_t row = e / d;
    const int64_t m = row / R;
    const float* cs[3] = {cq, ck, cv};
    const float ths[3] = {th_q[m], th_k[m], th_v[m]};
    float rate[3];
#pragma unroll
    for (int q = 0; q < 3; ++q) {
        const float vth = ths[q];
        float v = 0.0f, cnt = 0.0f, s;
        for (int32_t t = 0; t < T; ++t) {
            v = lif_upd(v, cs[q][(int64_t)t * total + e], leak, vth, &s);
            cnt = __fadd_rn(cnt, s);
        }
        rate[q] = __fdiv_rn(cnt, (float)T);
    }
    const int64_t pe = pos_per_member ? e : e % ((int64_t)R * d);
    X[e] = __fadd_rn(__fdiv_rn(__fadd_rn(__fadd_rn(rate[0], rate[1]), rate[2]), 3.0f), pos[pe]);
}

// One head of multihead_attention_once for one member per workgroup
// (snn_self_attention_heads.py:54-70 with row_softmax_lif): K, V (and Q) of
// the member's R tokens staged in LDS (dynamic, sized for R and hd, so that
// several workgroups share a CU); each wave takes groups of RP = min(4, 64 /
// hd) query rows.  Per row lane j is key neuron j: h_j = beta (q_i . k_j),
// normalised by max |h| + 1e-6, n_iter LIF steps with the inhibition g_inh *
// (sum of counts), p_j = count_j / (sum count + 1e-6) into the wave's LDS
// rows; then out_i = p @ V for the group's RP rows at once, lane rr * hd + c
// summing row rr's channel c over j in index order.
constexpr int kSaWaves = 4;
constexpr int kSaMaxR = 64, kSaMaxHd = 64, kSaMaxRP = 4;
constexpr int kSaPP = kSaMaxR + 1;  // pitch of a wave's p rows (rows on distinct banks)
static size_t sa_lds_bytes(int32_t R, int32_t hd) {
    return (3 * (size_t)R * (hd + 1) + (size_t)kSaWaves * kSaMaxRP * kSaPP) * sizeof(float);
}
__global__ __launch_bounds__(kSaWaves * 64) void k_sa_attention(
        const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
        int32_t ld, int32_t R, int32_t H, int32_t hd, const float* __restrict__ beta,
        const float* __restrict__ vth, float g_inh, float leak, int32_t n_iter,
        float* __restrict__ out) {
    extern __shared__ float sa_lds[];
    const int pitch = hd + 1;
    float* qs = sa_lds;
    float* ks = qs + R * pitch;
    float* vs = ks + R * pitch;
    const int32_t m = blockIdx.x / H, h = blockIdx.x % H;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    float* ps = vs + R * pitch + w * (kSaMaxRP * kSaPP);
    const int64_t row0 = (int64_t)m * R;
    for (int i = threadIdx.x; i < R * hd; i += kSaWaves * 64) {
        const int r = i / hd, c = i % hd;
        const int64_t g = (row0 + r) * ld + (int64_t)h * hd + c;
        qs[r * pitch + c] = Q[g];
        ks[r * pitch + c] = K[g];
        vs[r * pitch + c] = V[g];
    }
    __syncthreads();
    const float b = beta[m], th = vth[m];
    const bool key = lane < R;
    const int RP = min(kSaMaxRP, 64 / hd);
    const int rr = lane / hd, cc = lane - rr * hd;  // p @ V: row rr of the group, channel cc
    for (int i0 = w * RP; i0 < R; i0 += kSaWaves * RP) {
        const int nr = min(RP, R - i0);
        // the group's rows side by side (rows past R repeat row R - 1 and are
        // not stored): their wave reductions are independent chains
        float hn[kSaMaxRP], u[kSaMaxRP], cnt[kSaMaxRP];
        {
            float sd[kSaMaxRP];
#pragma unroll
            for (int q = 0; q < kSaMaxRP; ++q) sd[q] = 0.0f;
            if (key) {
                for (int c = 0; c < hd; ++c) {
                    const float kv = ks[lane * pitch + c];
#pragma unroll
                    for (int q = 0; q < kSaMaxRP; ++q)
                        sd[q] = __fadd_rn(sd[q], __fmul_rn(qs[min(i0 + q, R - 1) * pitch + c], kv));
                }
            }
#pragma unroll
            for (int q = 0; q < kSaMaxRP; ++q) {
                const float hj = key ? __fmul_rn(b, sd[q]) : 0.0f;
                const float den = __fadd_rn(wmax(key ? fabsf(hj) : 0.0f), 1e-6f);
                hn[q] = __fdiv_rn(hj, den);
                u[q] = 0.0f;
                cnt[q] = 0.0f;
            }
        }
        for (int it = 0; it < n_iter; ++it) {
#pragma unroll
            for (int q = 0; q < kSaMaxRP; ++q) {
                const float G = wsum(key ? cnt[q] : 0.0f);  // integer counts: exact in any order
                const float inh = __fmul_rn(g_inh, G);
                float sp;
                u[q] = lif_upd(u[q], __fsub_rn(hn[q], inh), leak, th, &sp);
                cnt[q] = __fadd_rn(cnt[q], sp);
            }
        }
#pragma unroll
        for (int q = 0; q < kSaMaxRP; ++q) {
            const float tot = wsum(key ? cnt[q] : 0.0f);
            if (key && q < nr) ps[q * kSaPP + lane] = __fdiv_rn(cnt[q], __fadd_rn(tot, 1e-6f));
        }
        // the group's weights are read by other lanes of this wave only
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
        if (rr < nr) {
            float s = 0.0f;
            for (int j = 0; j < R; ++j) s = __fadd_rn(s, __fmul_rn(ps[rr * kSaPP + j], vs[j * pitch + cc]));
            out[(row0 + i0 + rr) * ld + (int64_t)h * hd + cc] = s;
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }
}

// lif_single of ffn_once (snn_self_attention_heads.py:79-83): per row,
// act = c / max(max |c|, 1e-6) >= vth.  One wave per row.
__global__ __launch_bounds__(256) void k_sa_ffn_spike(const float* __restrict__ c, int64_t M,
                                                      int32_t d, int32_t R,
                                                      const float* __restrict__ vth,
                                                      float* __restrict__ act) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= M) return;  // whole wave
    const float* cr = c + row * d;
    float mx = 0.0f;
    for (int32_t j = lane; j < d; j += 64) mx = fmaxf(mx, fabsf(cr[j]));
    const float den = fmaxf(wmax(mx), 1e-6f);
    const float th = vth[row / R];
    for (int32_t j = lane; j < d; j += 64) act[row * d + j] = __fdiv_rn(cr[j], den) >= th ? 1.0f : 0.0f;
}

// x += y (the blocks' residual adds).
__global__ __launch_bounds__(256) void k_add_inplace(float* __restrict__ x,
                                                     const float* __restrict__ y, int64_t n) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e < n) x[e] = __fadd_rn(x[e], y[e]);
}

// jnp.mean(X, axis=0) per member: out[m, c] = (sum_i X[m R + i, c]) / R in
// index order.  One thread per (member, column).
__global__ __launch_bounds__(256) void k_sa_pool(const float* __restrict__ X, int64_t n,
                                                 int32_t R, int32_t d, float* __restrict__ out) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= n * d) return;
    const int64_t m = e / d;
    const int32_t c = (int32_t)(e % d);
    float s = 0.0f;
    for (int32_t i = 0; i < R; ++i) s = __fadd_rn(s, X[(m * R + i) * d + c]);
    out[e] = __fdiv_rn(s, (float)R);
}

// y[r, :] *= s[r] (logits * out_gain per member).
__global__ __launch_bounds__(256) void k_scale_rows(float* __restrict__ y, int64_t rows,
                                                    int32_t cols, const float* __restrict__ s) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e < rows * cols) y[e] = __fmul_rn(y[e], s[e / cols]);
}

static uint32_t blocks256(int64_t n) { return (uint32_t)((n + 255) / 256); }

}  // namespace hses

using namespace hses;

extern "C" int hses_softplus(const float* d_x, int64_t n, float* d_y, void* stream) {
    HSES_REQUIRE(n >= 0, "negative length");
    if (n == 0) return HSES_OK;
    HSES_REQUIRE(d_x && d_y, "NULL pointer");
    HSES_REQUIRE((n + 255) / 256 < (1ll << 31), "grid too large");
    hipLaunchKernelGGL(k_softplus, dim3(blocks256(n)), dim3(256), 0, (hipStream_t)stream, d_x, n, d_y);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_sa_encode(const float* d_cq, const float* d_ck, const float* d_cv, int32_t T,
                              int64_t M, int32_t d, int32_t rows_per_member, const float* d_th_q,
                              const float* d_th_k, const float* d_th_v, float tau_m,
                              const float* d_pos, int32_t pos_per_member, float* d_X,
                              void* stream) {
    HSES_REQUIRE(T >= 1 && M >= 0 && d >= 1 && rows_per_member >= 1, "bad sizes");
    HSES_REQUIRE(M % rows_per_member == 0, "rows are not a whole number of members");
    HSES_REQUIRE(tau_m > 0.0f, "tau_m must be > 0");
    if (M == 0) return HSES_OK;
    HSES_REQUIRE(d_cq && d_ck && d_cv && d_th_q && d_th_k && d_th_v && d_pos && d_X, "NULL pointer");
    HSES_REQUIRE(d_X != d_cq && d_X != d_ck && d_X != d_cv, "X must not alias the currents");
    HSES_REQUIRE((M * d + 255) / 256 < (1ll << 31), "grid too large");
    hipLaunchKernelGGL(k_sa_encode, dim3(blocks256(M * d)), dim3(256), 0, (hipStream_t)stream,
                       d_cq, d_ck, d_cv, T, M, d, rows_per_member, d_th_q, d_th_k, d_th_v,
                       1.0f / tau_m, d_pos,
                       pos_per_member, d_X);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_sa_attention(const float* d_q, const float* d_k, const float* d_v,
                                 int32_t ld, int64_t n, int32_t R, int32_t H, int32_t hd,
                                 const float* d_beta, const float* d_vth, float g_inh, float tau_m,
                                 int32_t n_iter, float* d_out, void* stream) {
    HSES_REQUIRE(n >= 0 && H >= 1 && n_iter >= 0, "bad sizes");
    HSES_REQUIRE(R >= 1 && R <= kSaMaxR, "tokens per member must be in [1, 64]");
    HSES_REQUIRE(hd >= 1 && hd <= kSaMaxHd, "head size must be in [1, 64]");
    HSES_REQUIRE(ld >= H * hd, "row stride smaller than the heads");
    HSES_REQUIRE(tau_m > 0.0f, "tau_m must be > 0");
    if (n == 0) return HSES_OK;
    HSES_REQUIRE(d_q && d_k && d_v && d_beta && d_vth && d_out, "NULL pointer");
    HSES_REQUIRE(d_out != d_q && d_out != d_k && d_out != d_v, "out must not alias q, k or v");
    HSES_REQUIRE(n * H < (1ll << 31), "grid too large");
    hipLaunchKernelGGL(k_sa_attention, dim3((uint32_t)(n * H)), dim3(kSaWaves * 64), sa_lds_bytes(R, hd),
                       (hipStream_t)stream, d_q, d_k, d_v, ld, R, H, hd, d_beta, d_vth, g_inh,
                       1.0f / tau_m, n_iter, d_out);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_sa_ffn_spike(const float* d_c, int64_t M, int32_t d, int32_t rows_per_member,
                                 const float* d_vth, float* d_act, void* stream) {
    HSES_REQUIRE(M >= 0 && d >= 1 && rows_per_member >= 1, "bad sizes");
    HSES_REQUIRE(M % rows_per_member == 0, "rows are not a whole number of members");
    if (M == 0) return HSES_OK;
    HSES_REQUIRE(d_c && d_vth && d_act, "NULL pointer");
    HSES_REQUIRE((M + 3) / 4 < (1ll << 31), "grid too large");
    hipLaunchKernelGGL(k_sa_ffn_spike, dim3((uint32_t)((M + 3) / 4)), dim3(256), 0,
                       (hipStream_t)stream, d_c, M, d, rows_per_member, d_vth, d_act);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_add_inplace(float* d_x, const float* d_y, int64_t n, void* stream) {
    HSES_REQUIRE(n >= 0, "negative length");
    if (n == 0) return HSES_OK;
    HSES_REQUIRE(d_x && d_y, "NULL pointer");
    HSES_REQUIRE((n + 255) / 256 < (1ll << 31), "grid too large");
    hipLaunchKernelGGL(k_add_inplace, dim3(blocks256(n)), dim3(256), 0, (hipStream_t)stream, d_x,
                       d_y, n);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_sa_pool(const float* d_X, int64_t n, int32_t R, int32_t d, float* d_out,
                            void* stream) {
    HSES_REQUIRE(n >= 0 && R >= 1 && d >= 1, "bad sizes");
    if (n == 0) return HSES_OK;
    HSES_REQUIRE(d_X && d_out, "NULL pointer");
    HSES_REQUIRE((n * d + 255) / 256 < (1ll << 31), "grid too large");
    hipLaunchKernelGGL(k_sa_pool, dim3(blocks256(n * d)), dim3(256), 0, (hipStream_t)stream, d_X,
                       n, R, d, d_out);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_scale_rows(float* d_y, int64_t rows, int32_t cols, const float* d_s,
                               void* stream) {
    HSES_REQUIRE(rows >= 0 && cols >= 1, "bad sizes");
    if (rows == 0) return HSES_OK;
    HSES_REQUIRE(d_y && d_s, "NULL pointer");
    HSES_REQUIRE((rows * cols + 255) / 256 < (1ll << 31), "grid too large");
    hipLaunchKernelGGL(k_scale_rows, dim3(blocks256(rows * cols)), dim3(256), 0,
                       (hipStream_t)stream, d_y, rows, cols, d_s);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}
