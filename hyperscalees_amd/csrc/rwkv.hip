// rwkv.hip -- RWKV-7 components of burn_impl/hyperscalees-models/src/llm.rs on the
// GPU: layer norm, group norm, the token-shift mix of TimeMixing/ChannelMixing,
// relu^2, and the rwkv7_inner_loop state recurrence (WKV-7), batched over
// sequences (one sequence per population member and sample).
//
// Every routine keeps the reference's per-element operation order with each
// operation rounded separately (built with -ffp-contract=off); reductions run
// over 64-lane waves, so their association differs from the reference's.  Two
// exceptions, both in TimeMixing's per-step work, which the recurrence kernel
// does for every element and step: the state update's multiply-adds are fused,
// and the gates use the hardware's exp2 / log2 / reciprocal / reciprocal-root
// instructions (about an ulp each) in place of libm-accurate routines.
#include <math.h>

#include <type_traits>

#include "runtime.h"

namespace hses {

// Round-to-nearest-even f32 -> bf16 bits (the rounding the bf16 MFMA operands get).
__device__ __forceinline__ uint16_t f2bf_rne(float f) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    return (uint16_t)__builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){f, 0.0f}, bf16x2_t));
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}

// Sum over the 64 lanes of a wave, the same bits in every lane (each exchange
// pairs lanes symmetrically and the adds commute): within rows of 16 lanes by
// DPP (quad swaps, then the half-row and row mirrors), across rows by the
// permlane16 and permlane32 swaps.  No LDS traffic.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm 1,0,3,2
    v += dpp_f<0x4E>(v);   // quad_perm 2,3,0,1
    v += dpp_f<0x141>(v);  // row_half_mirror: the other quad of the half-row
    v += dpp_f<0x140>(v);  // row_mirror: the other half-row
    const uint32_t u = __float_as_uint(v);
    const auto p16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    v = __uint_as_float(p16[0]) + __uint_as_float(p16[1]);  // rows 0+1 | 2+3
    const uint32_t w = __float_as_uint(v);
    const auto p32 = __builtin_amdgcn_permlane32_swap(w, w, false, false);
    return __uint_as_float(p32[0]) + __uint_as_float(p32[1]);
}

// TimeMixing's gate algebra on the hardware's transcendental instructions.
// Every kernel that forms a gate calls these, so the fused and unfused paths
// agree bit for bit.
__device__ __forceinline__ float exp_hw(float x) {
    return __builtin_amdgcn_exp2f(x * 1.44269504088896341f);
}
__device__ __forceinline__ float sigmoid_hw(float z) { return __builtin_amdgcn_rcpf(1.0f + exp_hw(-z)); }
// ln(1 + e^x), x itself above 20
__device__ __forceinline__ float softplus_hw(float x) {
    return x > 20.0f ? x : 0.693147180559945309f * __builtin_amdgcn_logf(1.0f + exp_hw(x));
}
// the recurrence's decay exp(-exp(w))
__device__ __forceinline__ float decay_hw(float w) { return exp_hw(-exp_hw(w)); }
// 1 / max(sqrt(ss), 1e-12): the kk normalisation
__device__ __forceinline__ float inv_norm_hw(float ss) {
    const float n = __builtin_amdgcn_sqrtf(ss);
    return __builtin_amdgcn_rcpf(n < 1e-12f ? 1e-12f : n);
}

// llm.rs:66-83: y = (x - mean) / sqrt(E[x^2] - mean^2 + eps) * w + b per row.
// One wave per row.
__global__ __launch_bounds__(256) void k_layer_norm(const float* __restrict__ x, int64_t rows,
                                                    int32_t C, const float* __restrict__ w,
                                                    const float* __restrict__ b, float eps,
                                                    float* __restrict__ y) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;  // whole wave
    const float* xr = x + row * C;
    float s = 0.0f, s2 = 0.0f;
    for (int32_t c = lane; c < C; c += 64) {
        const float v = xr[c];
        s = s + v;
        s2 = s2 + v * v;
    }
    const float mean = wave_sum(s) / (float)C;
    const float var = wave_sum(s2) / (float)C - mean * mean;
    const float sd = sqrtf(var + eps);
    for (int32_t c = lane; c < C; c += 64) y[row * C + c] = (xr[c] - mean) / sd * w[c] + b[c];
}

// llm.rs:97-150 (GroupNorm): x (n, C, L); group g of row i is channels
// [g C/G, (g+1) C/G) at all L positions; y = w[c] * (x - mean) / sqrt(var + eps)
// + b[c].  One wave per (row, group).
__global__ __launch_bounds__(256) void k_group_norm(const float* __restrict__ x, int64_t n,
                                                    int32_t C, int32_t L, int32_t G,
                                                    const float* __restrict__ w,
                                                    const float* __restrict__ b, float eps,
                                                    float* __restrict__ y) {
    const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (item >= n * G) return;  // whole wave
    const int64_t i = item / G;
    const int32_t g = (int32_t)(item - i * G), inner = C / G;
    const int64_t gsz = (int64_t)inner * L, base = (i * C + (int64_t)g * inner) * L;
    float s = 0.0f, s2 = 0.0f;
    for (int64_t e = lane; e < gsz; e += 64) {
        const float v = x[base + e];
        s = s + v;
        s2 = s2 + v * v;
    }
    const float mean = wave_sum(s) / (float)gsz;
    const float var = wave_sum(s2) / (float)gsz - mean * mean;
    const float isd = __builtin_amdgcn_rsqf(var + eps);  // as the fused TimeMixing output forms it
    for (int64_t e = lane; e < gsz; e += 64) {
        const int32_t c = g * inner + (int32_t)(e / L);
        y[base + e] = w[c] * ((x[base + e] - mean) * isd) + b[c];
    }
}

// The token shift of TimeMixing / ChannelMixing (llm.rs:200-205, 360-381) for
// n_mix mixing vectors at once: sx = [state, x[:-1]] (0 at a new start) - x,
// out[m] = x + sx * mix[m].  x (nseq, T, C), state (nseq, C), mix (n_mix, C),
// new_starts (nseq, T) or NULL, out (n_mix, nseq, T, C).
template <bool BF16OUT>
__global__ void k_token_shift_mix(const float* __restrict__ x, const float* __restrict__ state,
                                  const uint8_t* __restrict__ new_starts,
                                  const float* __restrict__ mix, int32_t n_mix, int64_t nseq,
                                  int32_t T, int32_t C, void* __restrict__ out) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = nseq * T * C;
    if (e >= total) return;
    const int32_t c = (int32_t)(e % C);
    const int64_t st = e / C;  // sequence * T + t
    const int32_t t = (int32_t)(st % T);
    const int64_t sq = st / T;
    float prev = t == 0 ? state[sq * C + c] : x[e - C];
    if (new_starts && new_starts[st]) prev = 0.0f;
    const float xv = x[e];
    const float sx = prev - xv;
    for (int32_t m = 0; m < n_mix; ++m) {
        const float v = xv + sx * mix[(int64_t)m * C + c];
        if constexpr (BF16OUT)
            static_cast<uint16_t*>(out)[(int64_t)m * total + e] = f2bf_rne(v);
        else
            static_cast<float*>(out)[(int64_t)m * total + e] = v;
    }
}

// The same for C % 4 == 0, four consecutive channels of one row per thread
// (16-byte loads, 16- or 8-byte stores, one row computation per four values).
template <bool BF16OUT>
__global__ void k_token_shift_mix4(const float* __restrict__ x, const float* __restrict__ state,
                                   const uint8_t* __restrict__ new_starts,
                                   const float* __restrict__ mix, int32_t n_mix, int64_t nseq,
                                   int32_t T, int32_t C, void* __restrict__ out) {
    const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = nseq * T * C;
    const int64_t e = q * 4;
    if (e >= total) return;
    const int32_t c4 = C >> 2;
    const int64_t st = q / c4;  // sequence * T + t
    const int32_t c = (int32_t)(q - st * c4) * 4;
    const int32_t t = (int32_t)(st % T);
    const int64_t sq = st / T;
    const float4 xv = *reinterpret_cast<const float4*>(x + e);
    float4 pv = t == 0 ? *reinterpret_cast<const float4*>(state + sq * C + c)
                       : *reinterpret_cast<const float4*>(x + e - C);
    if (new_starts && new_starts[st]) pv = float4{0.0f, 0.0f, 0.0f, 0.0f};
    const float sx0 = pv.x - xv.x, sx1 = pv.y - xv.y, sx2 = pv.z - xv.z, sx3 = pv.w - xv.w;
    for (int32_t m = 0; m < n_mix; ++m) {
        const float4 mv = *reinterpret_cast<const float4*>(mix + (int64_t)m * C + c);
        const float v0 = xv.x + sx0 * mv.x, v1 = xv.y + sx1 * mv.y;
        const float v2 = xv.z + sx2 * mv.z, v3 = xv.w + sx3 * mv.w;
        if constexpr (BF16OUT) {
            const uint2 pk{(uint32_t)f2bf_rne(v0) | ((uint32_t)f2bf_rne(v1) << 16),
                           (uint32_t)f2bf_rne(v2) | ((uint32_t)f2bf_rne(v3) << 16)};
            *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + (int64_t)m * total + e) = pk;
        } else {
            *reinterpret_cast<float4*>(static_cast<float*>(out) + (int64_t)m * total + e) =
                float4{v0, v1, v2, v3};
        }
    }
}

// llm.rs:206: relu(x)^2, in place.
__global__ void k_relu_sq(float* __restrict__ x, int64_t n) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n) return;
    const float z = x[e] > 0.0f ? x[e] : 0.0f;
    x[e] = z * z;
}

// llm.rs:235-300 (rwkv7_inner_loop) for nseq sequences: r, w, k, v, a, b
// (nseq, T, H, S); s_in / s_out (nseq, H, S, S); out (nseq, T, H, S);
// new_starts (nseq, T) or NULL.  One wave per (sequence, head), S <= 64: lane i
// holds row i of the head's state.  Per step the six vectors are staged in the
// wave's LDS slice (decay w -> exp(-exp(w)) on the way, by the hardware's exp2)
// and read as broadcasts; then sa_i = sum_j s_ij a_j, s_ij = ((s_ij w_j) + v_i k_j) + sa_i b_j,
// out_i = sum_j s_ij r_j, all sums in ascending j, each multiply-add fused
// (one rounding where the reference rounds the product and the sum: at most
// an ulp per operation apart; the kernel is bound by these vector operations,
// 5 per state element and step instead of 9).  s_out is the state after
// the last step t < length (s_in when length == 0).  s_in NULL: the zero
// state; s_out NULL: the final state is not stored.
// With POST the output row is TimeMixing's next three steps instead
// (llm.rs:455-470): y = (GroupNorm_head(out) + (sum_s r k r_k) v) g, with
// the group statistics and the readout sum formed exactly as k_group_norm and
// k_tm_post form them (the same per-lane terms and wave reductions), so the
// result equals the unfused chain bit for bit.
struct WkvPost {
    const float* g;
    const float* ln_w;
    const float* ln_b;
    const float* r_k;
    float eps;
    int32_t bf16_out;  // write the output rows as bf16 (nearest even)
};

// With GATES (and POST) the step's vectors are formed in the staging from
// TimeMixing's raw projections exactly as k_tm_gates_kk forms them: w is the
// decay branch's w2 output, a the rate branch's a2 output, k and v the raw key
// and value, and the per-head kk norm is a wave sum, so nothing between the
// projections and the output goes through memory.
struct WkvGates {
    const float* v2o;      // value branch's v2 output, NULL at the first layer
    const float* v_first;  // (with v2o)
    const float* w0;
    const float* a0;
    const float* v0;
    const float* k_k;
    const float* k_a;
};

template <int S, bool POST, bool GATES>
__global__ __launch_bounds__(256) void k_wkv7(const float* __restrict__ r, const float* __restrict__ w,
                                              const float* __restrict__ k, const float* __restrict__ v,
                                              const float* __restrict__ a, const float* __restrict__ b,
                                              const float* __restrict__ s_in,
                                              const uint8_t* __restrict__ new_starts, int64_t nseq,
                                              int32_t T, int32_t H, int32_t length,
                                              float* __restrict__ out, float* __restrict__ s_out,
                                              WkvPost post, WkvGates gt) {
    __shared__ __align__(16) float stage[4][6][64];
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t item = (int64_t)blockIdx.x * 4 + wv;
    if (item >= nseq * H) return;  // whole wave
    const int64_t sq = item / H;
    const int32_t h = (int32_t)(item - sq * H);
    const bool row_ok = lane < S;
    const int i = row_ok ? lane : 0;
    const int64_t sbase = (sq * H + h) * (int64_t)S * S + (int64_t)i * S;
    float s[S];
#pragma unroll
    for (int j = 0; j < S; ++j) s[j] = s_in ? s_in[sbase + j] : 0.0f;
    float (*st)[64] = stage[wv];
    // this lane's elements of the step's six vectors (and the gate g with POST),
    // loaded one step ahead so their latency overlaps the previous step's work
    float nr = 0.0f, nw = 0.0f, nk = 0.0f, nv = 0.0f, na = 0.0f, nb = 0.0f, ng = 0.0f;
    float nv2 = 0.0f, nvf = 0.0f;
    uint8_t nns = 0;  // the step's new-start flag
    const int32_t cc = h * S + i;  // this lane's channel
    float w0c = 0.0f, a0c = 0.0f, v0c = 0.0f, kkc = 0.0f, kac = 0.0f;
    if constexpr (GATES) {
        w0c = gt.w0[cc];
        a0c = gt.a0[cc];
        v0c = gt.v2o ? gt.v0[cc] : 0.0f;
        kkc = gt.k_k[cc];
        kac = gt.k_a[cc];
    }
    auto fetch = [&](int32_t t) {
        const int64_t o = ((sq * T + t) * H + h) * (int64_t)S + i;
        if (new_starts) nns = new_starts[sq * T + t];
        nr = r[o];
        nw = w[o];
        nk = k[o];
        nv = v[o];
        na = a[o];
        if constexpr (GATES) {
            if (gt.v2o) {
                nv2 = gt.v2o[o];
                nvf = gt.v_first[o];
            }
        } else {
            nb = b[o];
        }
        if constexpr (POST) ng = post.g[o];
    };
    fetch(0);
    for (int32_t t = 0; t < T; ++t) {
        if (nns) {
#pragma unroll
            for (int j = 0; j < S; ++j) s[j] = 0.0f;
        }
        const int64_t o = ((sq * T + t) * H + h) * (int64_t)S;
        const float gcur = ng;
        if constexpr (GATES) {
            // k_tm_gates_kk's per-element algebra (same operations, same wave sum)
            const float wv = -softplus_hw(-(w0c + nw)) - 0.5f;
            const float av = sigmoid_hw(a0c + na);
            float vv = nv;
            if (gt.v2o) {
                const float sg = sigmoid_hw(v0c + nv2);
                vv = vv + (nvf - vv) * sg;
            }
            const float kk2 = row_ok ? nk * kkc : 0.0f;
            const float kk = kk2 * inv_norm_hw(wave_sum(kk2 * kk2));
            if (row_ok) {
                st[0][lane] = nr;
                st[1][lane] = decay_hw(wv);
                st[2][lane] = nk * (kac * (av - 1.0f) + 1.0f);
                st[3][lane] = vv;
                st[4][lane] = -kk;
                st[5][lane] = kk * av;
            }
        } else if (row_ok) {
            st[0][lane] = nr;
            st[1][lane] = decay_hw(nw);
            st[2][lane] = nk;
            st[3][lane] = nv;
            st[4][lane] = na;
            st[5][lane] = nb;
        }
        if (t + 1 < T) fetch(t + 1);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const float vi = st[3][i];
        float sa = 0.0f;
#pragma unroll
        for (int j = 0; j < S; ++j) sa = __builtin_fmaf(s[j], st[4][j], sa);
#pragma unroll
        for (int j = 0; j < S; ++j)
            s[j] = __builtin_fmaf(sa, st[5][j], __builtin_fmaf(vi, st[2][j], s[j] * st[1][j]));
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < S; ++j) acc = __builtin_fmaf(s[j], st[0][j], acc);
        if constexpr (POST) {
            const float x1 = row_ok ? acc : 0.0f;
            const float mean = wave_sum(0.0f + x1) / (float)S;
            const float var = wave_sum(0.0f + x1 * x1) / (float)S - mean * mean;
            const float isd = __builtin_amdgcn_rsqf(var + post.eps);
            const int32_t c = h * S + i;
            const float rk = wave_sum(row_ok ? st[0][i] * st[2][i] * post.r_k[c] : 0.0f);
            if (row_ok) {
                const float gn = post.ln_w[c] * ((acc - mean) * isd) + post.ln_b[c];
                const float y = (gn + rk * vi) * gcur;
                if (post.bf16_out)
                    reinterpret_cast<uint16_t*>(out)[o + lane] = f2bf_rne(y);
                else
                    out[o + lane] = y;
            }
        } else {
            if (row_ok) out[o + lane] = acc;
        }
        if (t == length - 1 && row_ok && s_out) {
#pragma unroll
            for (int j = 0; j < S; ++j) s_out[sbase + j] = s[j];
        }
        // the next step's staging overwrites st: every lane has read it
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    if (length <= 0 && row_ok && s_out) {
#pragma unroll
        for (int j = 0; j < S; ++j) s_out[sbase + j] = s_in ? s_in[sbase + j] : 0.0f;
    }
}

// Activations of TimeMixing's low-rank branches, in place: kind 0 tanh
// (w1, v1, a1 outputs), kind 1 sigmoid (g1 output).
__global__ void k_rwkv_act(float* __restrict__ x, int64_t n, int32_t kind) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n) return;
    const float z = x[e];
    x[e] = kind == 0 ? tanhf(z) : 1.0f / (1.0f + expf(-z));
}


// TimeMixing gates (llm.rs:388-408), per element of (rows, C):
//   w = -softplus(-(w0 + w2o)) - 0.5 (written over w2o);
//   a = sigmoid(a0 + a2o) (written over a2o);
//   v2o != NULL (layers after the first): v = v + (v_first - v) * sigmoid(v0 + v2o).
__global__ void k_tm_gates(float* __restrict__ w2o, float* __restrict__ a2o,
                           const float* __restrict__ v2o, float* __restrict__ v,
                           const float* __restrict__ v_first, const float* __restrict__ w0,
                           const float* __restrict__ a0, const float* __restrict__ v0, int64_t n,
                           int32_t C) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n) return;
    const int32_t c = (int32_t)(e % C);
    w2o[e] = -softplus_hw(-(w0[c] + w2o[e])) - 0.5f;
    a2o[e] = sigmoid_hw(a0[c] + a2o[e]);
    if (v2o) {
        const float sg = sigmoid_hw(v0[c] + v2o[e]);
        v[e] = v[e] + (v_first[e] - v[e]) * sg;
    }
}

// TimeMixing's kk normalisation (llm.rs:414-426) per (row, head), one wave
// each (S <= 64 lanes): kk = k k_k / max(||k k_k||, 1e-12); a_i = -kk;
// b_i = kk a; k = k (k_a (a - 1) + 1) in place.
__global__ __launch_bounds__(256) void k_tm_kk(float* __restrict__ k, const float* __restrict__ k_k,
                                               const float* __restrict__ k_a,
                                               const float* __restrict__ a, int64_t rows,
                                               int32_t H, int32_t S, float* __restrict__ ai,
                                               float* __restrict__ bi) {
    const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (item >= rows * H) return;  // whole wave
    const int64_t row = item / H;
    const int32_t h = (int32_t)(item - row * H), C = H * S, c = h * S + lane;
    const bool ok = lane < S;
    const int64_t o = row * C + c;
    const float kv = ok ? k[o] : 0.0f;
    const float kk2 = ok ? kv * k_k[c] : 0.0f;
    const float inv = inv_norm_hw(wave_sum(kk2 * kk2));
    if (!ok) return;
    const float kk = kk2 * inv, av = a[o];
    ai[o] = -kk;
    bi[o] = kk * av;
    k[o] = kv * (k_a[c] * (av - 1.0f) + 1.0f);
}

// TimeMixing's readout and gate (llm.rs:455-470) per (row, head), one wave
// each: x = (gn + (sum_s r k r_k) v) g, with gn the group-normed recurrence
// output.  Written over gn.
__global__ __launch_bounds__(256) void k_tm_post(float* __restrict__ gn, const float* __restrict__ r,
                                                 const float* __restrict__ k,
                                                 const float* __restrict__ v,
                                                 const float* __restrict__ g,
                                                 const float* __restrict__ r_k, int64_t rows,
                                                 int32_t H, int32_t S) {
    const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (item >= rows * H) return;  // whole wave
    const int64_t row = item / H;
    const int32_t h = (int32_t)(item - row * H), C = H * S, c = h * S + lane;
    const bool ok = lane < S;
    const int64_t o = row * C + c;
    const float sum = wave_sum(ok ? r[o] * k[o] * r_k[c] : 0.0f);
    if (ok) gn[o] = (gn[o] + sum * v[o]) * g[o];
}

// The LM's embedding lookup fused with ln0 (rwkv7.py:189-192, 227): row i is
// emb[tok[i]] layer-normed.  A token outside [0, V) reads nothing and gives a
// row of NaN.  One wave per row.
__global__ __launch_bounds__(256) void k_embed_layer_norm(const int32_t* __restrict__ tok,
                                                          int64_t rows,
                                                          const float* __restrict__ emb,
                                                          int32_t V, int32_t C,
                                                          const float* __restrict__ w,
                                                          const float* __restrict__ b, float eps,
                                                          float* __restrict__ y) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;  // whole wave
    const int32_t t = tok[row];
    float* yr = y + row * C;
    if (t < 0 || t >= V) {
        for (int32_t c = lane; c < C; c += 64) yr[c] = __builtin_nanf("");
        return;
    }
    const float* xr = emb + (int64_t)t * C;
    float s = 0.0f, s2 = 0.0f;
    for (int32_t c = lane; c < C; c += 64) {
        const float v = xr[c];
        s = s + v;
        s2 = s2 + v * v;
    }
    const float mean = wave_sum(s) / (float)C;
    const float var = wave_sum(s2) / (float)C - mean * mean;
    const float sd = sqrtf(var + eps);
    for (int32_t c = lane; c < C; c += 64) yr[c] = (xr[c] - mean) / sd * w[c] + b[c];
}

// The block's residual add fused with the LayerNorm that follows it
// (rwkv7.py:243-252, 194-196): x += d in place, then y = LayerNorm(x).
// One wave per row; each lane keeps its sums of the updated values.
__global__ __launch_bounds__(256) void k_add_layer_norm(float* __restrict__ x,
                                                        const float* __restrict__ d, int64_t rows,
                                                        int32_t C, const float* __restrict__ w,
                                                        const float* __restrict__ b, float eps,
                                                        float* __restrict__ y) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;  // whole wave
    float* xr = x + row * C;
    const float* dr = d + row * C;
    float s = 0.0f, s2 = 0.0f;
    for (int32_t c = lane; c < C; c += 64) {
        const float v = xr[c] + dr[c];
        xr[c] = v;
        s = s + v;
        s2 = s2 + v * v;
    }
    const float mean = wave_sum(s) / (float)C;
    const float var = wave_sum(s2) / (float)C - mean * mean;
    const float sd = sqrtf(var + eps);
    float* yr = y + row * C;
    for (int32_t c = lane; c < C; c += 64) yr[c] = (xr[c] - mean) / sd * w[c] + b[c];
}

// k_add_layer_norm for C = 256 NV: lane l holds channels 256 j + 4 l .. + 3
// (j < NV) in registers, read and written with 16-byte accesses.
template <int NV>
__global__ __launch_bounds__(256) void k_add_layer_norm4(float* __restrict__ x,
                                                         const float* __restrict__ d, int64_t rows,
                                                         const float* __restrict__ w,
                                                         const float* __restrict__ b, float eps,
                                                         float* __restrict__ y) {
    constexpr int C = 256 * NV;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;  // whole wave
    float4* xr = reinterpret_cast<float4*>(x + row * C);
    const float4* dr = reinterpret_cast<const float4*>(d + row * C);
    float4 v[NV];
    float s = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const float4 a = xr[64 * j + lane], e = dr[64 * j + lane];
        v[j] = float4{a.x + e.x, a.y + e.y, a.z + e.z, a.w + e.w};
        xr[64 * j + lane] = v[j];
        s = s + v[j].x;
        s = s + v[j].y;
        s = s + v[j].z;
        s = s + v[j].w;
        s2 = s2 + v[j].x * v[j].x;
        s2 = s2 + v[j].y * v[j].y;
        s2 = s2 + v[j].z * v[j].z;
        s2 = s2 + v[j].w * v[j].w;
    }
    const float mean = wave_sum(s) / (float)C;
    const float var = wave_sum(s2) / (float)C - mean * mean;
    const float sd = sqrtf(var + eps);
    float4* yr = reinterpret_cast<float4*>(y + row * C);
    const float4* w4 = reinterpret_cast<const float4*>(w);
    const float4* b4 = reinterpret_cast<const float4*>(b);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const float4 ww = w4[64 * j + lane], bb = b4[64 * j + lane];
        yr[64 * j + lane] = float4{(v[j].x - mean) / sd * ww.x + bb.x, (v[j].y - mean) / sd * ww.y + bb.y,
                                   (v[j].z - mean) / sd * ww.z + bb.z, (v[j].w - mean) / sd * ww.w + bb.w};
    }
}

// A block's residual add, the LayerNorm that reads it and the next module's
// token shift in one pass (llm.rs:66-83, 200-205, 360-381): one wave per
// sequence walks its T rows in order, so the previous row's normalised values
// are still in its registers when the row's mixes are formed; the next two
// rows' x and delta are loaded ahead.  Per row the arithmetic is that of
// k_add_layer_norm4 (ADD) followed by k_token_shift_mix4, element for element,
// so the mixes (and x) equal the two-kernel chain's bit for bit; without ADD the
// row is normalised as k_add_layer_norm4 normalises x + 0 and x is not written.
// y_last (or NULL) receives the normalised row length - 1 (the next shift state).
template <int NV, int NMIX, bool ADD, bool BF16OUT>
__global__ __launch_bounds__(256) void k_ln_shift(float* __restrict__ x, const float* __restrict__ d,
                                                  int64_t nseq, int32_t T,
                                                  const float* __restrict__ w,
                                                  const float* __restrict__ b, float eps,
                                                  const float* __restrict__ state,
                                                  const uint8_t* __restrict__ new_starts,
                                                  const float* __restrict__ mix,
                                                  void* __restrict__ out,
                                                  float* __restrict__ y_last, int32_t length) {
    constexpr int C = 256 * NV;
    const int64_t q = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (q >= nseq) return;  // whole wave
    const int64_t plane = nseq * T * C;  // elements of one mix's output
    float4 wv[NV], bv[NV], mv[NMIX][NV], prev[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        wv[j] = reinterpret_cast<const float4*>(w)[64 * j + lane];
        bv[j] = reinterpret_cast<const float4*>(b)[64 * j + lane];
        prev[j] = reinterpret_cast<const float4*>(state + q * C)[64 * j + lane];
#pragma unroll
        for (int m = 0; m < NMIX; ++m) mv[m][j] = reinterpret_cast<const float4*>(mix + (int64_t)m * C)[64 * j + lane];
    }
    float4 xa[3][NV], da[3][NV];  // rows t, t + 1, t + 2
    auto load = [&](int32_t t, float4 (&xo)[NV], float4 (&dout)[NV]) {
        const int64_t r = q * T + (t < T ? t : T - 1);  // past the end: the last row again
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            xo[j] = reinterpret_cast<const float4*>(x + r * C)[64 * j + lane];
            if constexpr (ADD) dout[j] = reinterpret_cast<const float4*>(d + r * C)[64 * j + lane];
        }
    };
    load(0, xa[0], da[0]);
    load(1, xa[1], da[1]);
    for (int32_t t = 0; t < T; ++t) {
        load(t + 2, xa[2], da[2]);
        const int64_t r = q * T + t;
        float4 v[NV];
        float s = 0.0f, s2 = 0.0f;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const float4 a = xa[0][j];
            if constexpr (ADD) {
                const float4 e = da[0][j];
                v[j] = float4{a.x + e.x, a.y + e.y, a.z + e.z, a.w + e.w};
                reinterpret_cast<float4*>(x + r * C)[64 * j + lane] = v[j];
            } else {
                v[j] = float4{a.x + 0.0f, a.y + 0.0f, a.z + 0.0f, a.w + 0.0f};
            }
            s = s + v[j].x;
            s = s + v[j].y;
            s = s + v[j].z;
            s = s + v[j].w;
            s2 = s2 + v[j].x * v[j].x;
            s2 = s2 + v[j].y * v[j].y;
            s2 = s2 + v[j].z * v[j].z;
            s2 = s2 + v[j].w * v[j].w;
        }
        const float mean = wave_sum(s) / (float)C;
        const float var = wave_sum(s2) / (float)C - mean * mean;
        const float sd = sqrtf(var + eps);
        const bool fresh = new_starts && new_starts[r];
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const float4 ww = wv[j], bb = bv[j];
            const float4 y{(v[j].x - mean) / sd * ww.x + bb.x, (v[j].y - mean) / sd * ww.y + bb.y,
                           (v[j].z - mean) / sd * ww.z + bb.z, (v[j].w - mean) / sd * ww.w + bb.w};
            if (y_last && t == length - 1) reinterpret_cast<float4*>(y_last + q * C)[64 * j + lane] = y;
            const float4 pv = fresh ? float4{0.0f, 0.0f, 0.0f, 0.0f} : prev[j];
            const float sx0 = pv.x - y.x, sx1 = pv.y - y.y, sx2 = pv.z - y.z, sx3 = pv.w - y.w;
            const int64_t e = r * C + 4 * (64 * j + lane);
#pragma unroll
            for (int m = 0; m < NMIX; ++m) {
                const float4 mm = mv[m][j];
                const float v0 = y.x + sx0 * mm.x, v1 = y.y + sx1 * mm.y;
                const float v2 = y.z + sx2 * mm.z, v3 = y.w + sx3 * mm.w;
                if constexpr (BF16OUT) {
                    const uint2 pk{(uint32_t)f2bf_rne(v0) | ((uint32_t)f2bf_rne(v1) << 16),
                                   (uint32_t)f2bf_rne(v2) | ((uint32_t)f2bf_rne(v3) << 16)};
                    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + (int64_t)m * plane + e) = pk;
                } else {
                    *reinterpret_cast<float4*>(static_cast<float*>(out) + (int64_t)m * plane + e) =
                        float4{v0, v1, v2, v3};
                }
            }
            prev[j] = y;
        }
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            xa[0][j] = xa[1][j];
            xa[1][j] = xa[2][j];
            if constexpr (ADD) {
                da[0][j] = da[1][j];
                da[1][j] = da[2][j];
            }
        }
    }
}

// k_tm_gates and k_tm_kk in one pass, per (row, head), one wave each: the
// same per-element operations (a stays in registers instead of memory), so the
// outputs equal the two-kernel chain bit for bit.
__global__ __launch_bounds__(256) void k_tm_gates_kk(
    float* __restrict__ w2o, const float* __restrict__ a2o, const float* __restrict__ v2o,
    float* __restrict__ v, const float* __restrict__ v_first, const float* __restrict__ w0,
    const float* __restrict__ a0, const float* __restrict__ v0, float* __restrict__ k,
    const float* __restrict__ k_k, const float* __restrict__ k_a, int64_t rows, int32_t H,
    int32_t S, float* __restrict__ ai, float* __restrict__ bi) {
    const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (item >= rows * H) return;  // whole wave
    const int64_t row = item / H;
    const int32_t h = (int32_t)(item - row * H), C = H * S, c = h * S + lane;
    const bool ok = lane < S;
    const int64_t o = row * C + c;
    float av = 0.0f, kv = 0.0f;
    if (ok) {
        w2o[o] = -softplus_hw(-(w0[c] + w2o[o])) - 0.5f;
        av = sigmoid_hw(a0[c] + a2o[o]);
        if (v2o) {
            const float sg = sigmoid_hw(v0[c] + v2o[o]);
            v[o] = v[o] + (v_first[o] - v[o]) * sg;
        }
        kv = k[o];
    }
    const float kk2 = ok ? kv * k_k[c] : 0.0f;
    const float inv = inv_norm_hw(wave_sum(kk2 * kk2));
    if (!ok) return;
    const float kk = kk2 * inv;
    ai[o] = -kk;
    bi[o] = kk * av;
    k[o] = kv * (k_a[c] * (av - 1.0f) + 1.0f);
}

}  // namespace hses

using namespace hses;

static uint32_t blocks_of(int64_t n, int per) { return (uint32_t)((n + per - 1) / per); }

extern "C" int hses_layer_norm(const float* d_x, int64_t rows, int32_t C, const float* d_w,
                               const float* d_b, float eps, float* d_y, void* stream) {
    HSES_REQUIRE(rows >= 0 && C >= 1, "bad sizes");
    if (rows == 0) return HSES_OK;
    HSES_REQUIRE(d_x && d_w && d_b && d_y, "NULL pointer");
    HSES_REQUIRE((rows + 3) / 4 < (1ll << 31), "grid too large");
    hipLaunchKernelGGL(k_layer_norm, dim3(blocks_of(rows, 4)), dim3(256), 0, (hipStream_t)stream,
                       d_x, rows, C, d_w, d_b, eps, d_y);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_group_norm(const float* d_x, int64_t n, int32_t C, int32_t L, int32_t G,
                               const float* d_w, const float* d_b, float eps, float* d_y,
                               void* stream) {
    HSES_REQUIRE(n >= 0 && C >= 1 && L >= 1 && G >= 1 && C % G == 0, "bad sizes (C % G != 0?)");
    if (n == 0) return HSES_OK;
    HSES_REQUIRE(d_x && d_w && d_b && d_y, "NULL pointer");
    HSES_REQUIRE((n * G + 3) / 4 < (1ll << 31), "grid too large");
    hipLaunchKernelGGL(k_group_norm, dim3(blocks_of(n * G, 4)), dim3(256), 0, (hipStream_t)stream,
                       d_x, n, C, L, G, d_w, d_b, eps, d_y);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_token_shift_mix(const float* d_x, const float* d_state,
                                    const uint8_t* d_new_starts, const float* d_mix, int32_t n_mix,
                                    int64_t nseq, int32_t T, int32_t C, void* d_out,
                                    int32_t out_fmt, void* stream) {
    HSES_REQUIRE(nseq >= 0 && T >= 1 && C >= 1 && n_mix >= 1, "bad sizes");
    HSES_REQUIRE(out_fmt == HSES_FMT_F32 || out_fmt == HSES_FMT_BF16, "out_fmt must be F32 or BF16");
    if (nseq == 0) return HSES_OK;
    HSES_REQUIRE(d_x && d_state && d_mix && d_out, "NULL pointer");
    const int64_t total = nseq * T * C;
    HSES_REQUIRE((total + 255) / 256 < (1ll << 31), "grid too large");
    const bool bf = out_fmt == HSES_FMT_BF16;
    const bool vec = C % 4 == 0 && reinterpret_cast<uintptr_t>(d_x) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(d_state) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(d_mix) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(d_out) % 16 == 0;
    if (vec)
        hipLaunchKernelGGL(bf ? k_token_shift_mix4<true> : k_token_shift_mix4<false>,
                           dim3(blocks_of(total / 4, 256)), dim3(256), 0, (hipStream_t)stream, d_x,
                           d_state, d_new_starts, d_mix, n_mix, nseq, T, C, d_out);
    else
        hipLaunchKernelGGL(bf ? k_token_shift_mix<true> : k_token_shift_mix<false>,
                           dim3(blocks_of(total, 256)), dim3(256), 0, (hipStream_t)stream, d_x,
                           d_state, d_new_starts, d_mix, n_mix, nseq, T, C, d_out);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_relu_sq(float* d_x, int64_t n, void* stream) {
    HSES_REQUIRE(n >= 0, "negative size");
    if (n == 0) return HSES_OK;
    HSES_REQUIRE(d_x, "NULL pointer");
    HSES_REQUIRE((n + 255) / 256 < (1ll << 31), "grid too large");
    hipLaunchKernelGGL(k_relu_sq, dim3(blocks_of(n, 256)), dim3(256), 0, (hipStream_t)stream, d_x, n);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

template <bool POST, bool GATES = false>
static int launch_wkv7(const float* d_r, const float* d_w, const float* d_k, const float* d_v,
                       const float* d_a, const float* d_b, const float* d_s_in,
                       const uint8_t* d_new_starts, int64_t nseq, int32_t T, int32_t H, int32_t S,
                       int32_t length, float* d_out, float* d_s_out, WkvPost post, void* stream,
                       WkvGates gt = WkvGates{}) {
    HSES_REQUIRE((nseq * H + 3) / 4 < (1ll << 31), "grid too large");
    const dim3 g(blocks_of(nseq * H, 4)), blk(256);
    hipStream_t s = (hipStream_t)stream;
    if (S == 64)
        hipLaunchKernelGGL((k_wkv7<64, POST, GATES>), g, blk, 0, s, d_r, d_w, d_k, d_v, d_a, d_b,
                           d_s_in, d_new_starts, nseq, T, H, length, d_out, d_s_out, post, gt);
    else if (S == 32)
        hipLaunchKernelGGL((k_wkv7<32, POST, GATES>), g, blk, 0, s, d_r, d_w, d_k, d_v, d_a, d_b,
                           d_s_in, d_new_starts, nseq, T, H, length, d_out, d_s_out, post, gt);
    else
        hipLaunchKernelGGL((k_wkv7<16, POST, GATES>), g, blk, 0, s, d_r, d_w, d_k, d_v, d_a, d_b,
                           d_s_in, d_new_starts, nseq, T, H, length, d_out, d_s_out, post, gt);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_rwkv7_wkv(const float* d_r, const float* d_w, const float* d_k, const float* d_v,
                              const float* d_a, const float* d_b, const float* d_s_in,
                              const uint8_t* d_new_starts, int64_t nseq, int32_t T, int32_t H,
                              int32_t S, int32_t length, float* d_out, float* d_s_out,
                              void* stream) {
    HSES_REQUIRE(nseq >= 0 && T >= 1 && H >= 1, "bad sizes");
    HSES_REQUIRE(S == 16 || S == 32 || S == 64, "head size S must be 16, 32 or 64");
    HSES_REQUIRE(length >= 0 && length <= T, "length must be in [0, T]");
    if (nseq == 0) return HSES_OK;
    HSES_REQUIRE(d_r && d_w && d_k && d_v && d_a && d_b && d_out, "NULL pointer");
    HSES_REQUIRE(!d_s_out || d_s_out != d_s_in, "s_out must not alias s_in");
    return launch_wkv7<false>(d_r, d_w, d_k, d_v, d_a, d_b, d_s_in, d_new_starts, nseq, T, H, S,
                              length, d_out, d_s_out, WkvPost{}, stream);
}

extern "C" int hses_tm_wkv_post(const float* d_r, const float* d_w, const float* d_k,
                                const float* d_v, const float* d_a, const float* d_b,
                                const float* d_s_in, const uint8_t* d_new_starts, int64_t nseq,
                                int32_t T, int32_t H, int32_t S, int32_t length, const float* d_g,
                                const float* d_ln_w, const float* d_ln_b, float eps,
                                const float* d_r_k, void* d_out, int32_t out_fmt, float* d_s_out,
                                void* stream) {
    HSES_REQUIRE(out_fmt == HSES_FMT_F32 || out_fmt == HSES_FMT_BF16, "out_fmt must be F32 or BF16");
    HSES_REQUIRE(nseq >= 0 && T >= 1 && H >= 1, "bad sizes");
    HSES_REQUIRE(S == 16 || S == 32 || S == 64, "head size S must be 16, 32 or 64");
    HSES_REQUIRE(length >= 0 && length <= T, "length must be in [0, T]");
    if (nseq == 0) return HSES_OK;
    HSES_REQUIRE(d_r && d_w && d_k && d_v && d_a && d_b && d_out && d_g &&
                     d_ln_w && d_ln_b && d_r_k,
                 "NULL pointer");
    HSES_REQUIRE(!d_s_out || d_s_out != d_s_in, "s_out must not alias s_in");
    HSES_REQUIRE(d_out != d_r && d_out != d_k && d_out != d_v, "out must not alias r, k or v");
    return launch_wkv7<true>(d_r, d_w, d_k, d_v, d_a, d_b, d_s_in, d_new_starts, nseq, T, H, S,
                             length, static_cast<float*>(d_out), d_s_out,
                             WkvPost{d_g, d_ln_w, d_ln_b, d_r_k, eps, out_fmt == HSES_FMT_BF16},
                             stream);
}

extern "C" int hses_rwkv_act(float* d_x, int64_t n, int32_t kind, void* stream) {
    HSES_REQUIRE(n >= 0 && (kind == 0 || kind == 1), "bad arguments (kind 0 tanh, 1 sigmoid)");
    if (n == 0) return HSES_OK;
    HSES_REQUIRE(d_x, "NULL pointer");
    HSES_REQUIRE((n + 255) / 256 < (1ll << 31), "grid too large");
    hipLaunchKernelGGL(k_rwkv_act, dim3(blocks_of(n, 256)), dim3(256), 0, (hipStream_t)stream, d_x, n,
                       kind);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_tm_gates(float* d_w2o, float* d_a2o, const float* d_v2o, float* d_v,
                             const float* d_v_first, const float* d_w0, const float* d_a0,
                             const float* d_v0, int64_t rows, int32_t C, void* stream) {
    HSES_REQUIRE(rows >= 0 && C >= 1, "bad sizes");
    if (rows == 0) return HSES_OK;
    HSES_REQUIRE(d_w2o && d_a2o && d_w0 && d_a0, "NULL pointer");
    HSES_REQUIRE(!d_v2o || (d_v && d_v_first && d_v0), "NULL pointer (v branch)");
    const int64_t n = rows * C;
    HSES_REQUIRE((n + 255) / 256 < (1ll << 31), "grid too large");
    hipLaunchKernelGGL(k_tm_gates, dim3(blocks_of(n, 256)), dim3(256), 0, (hipStream_t)stream, d_w2o,
                       d_a2o, d_v2o, d_v, d_v_first, d_w0, d_a0, d_v0, n, C);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_tm_kk(float* d_k, const float* d_k_k, const float* d_k_a, const float* d_a,
                          int64_t rows, int32_t H, int32_t S, float* d_ai, float* d_bi,
                          void* stream) {
    HSES_REQUIRE(rows >= 0 && H >= 1 && S >= 1 && S <= 64, "bad sizes (S <= 64)");
    if (rows == 0) return HSES_OK;
    HSES_REQUIRE(d_k && d_k_k && d_k_a && d_a && d_ai && d_bi, "NULL pointer");
    HSES_REQUIRE((rows * H + 3) / 4 < (1ll << 31), "grid too large");
    hipLaunchKernelGGL(k_tm_kk, dim3(blocks_of(rows * H, 4)), dim3(256), 0, (hipStream_t)stream, d_k,
                       d_k_k, d_k_a, d_a, rows, H, S, d_ai, d_bi);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_tm_post(float* d_gn, const float* d_r, const float* d_k, const float* d_v,
                            const float* d_g, const float* d_r_k, int64_t rows, int32_t H,
                            int32_t S, void* stream) {
    HSES_REQUIRE(rows >= 0 && H >= 1 && S >= 1 && S <= 64, "bad sizes (S <= 64)");
    if (rows == 0) return HSES_OK;
    HSES_REQUIRE(d_gn && d_r && d_k && d_v && d_g && d_r_k, "NULL pointer");
    HSES_REQUIRE((rows * H + 3) / 4 < (1ll << 31), "grid too large");
    hipLaunchKernelGGL(k_tm_post, dim3(blocks_of(rows * H, 4)), dim3(256), 0, (hipStream_t)stream,
                       d_gn, d_r, d_k, d_v, d_g, d_r_k, rows, H, S);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_embed_layer_norm(const int32_t* d_tokens, int64_t rows, const float* d_emb,
                                     int32_t V, int32_t C, const float* d_w, const float* d_b,
                                     float eps, float* d_y, void* stream) {
    HSES_REQUIRE(rows >= 0 && V >= 1 && C >= 1, "bad sizes");
    if (rows == 0) return HSES_OK;
    HSES_REQUIRE(d_tokens && d_emb && d_w && d_b && d_y, "NULL pointer");
    HSES_REQUIRE((rows + 3) / 4 < (1ll << 31), "grid too large");
    hipLaunchKernelGGL(k_embed_layer_norm, dim3(blocks_of(rows, 4)), dim3(256), 0,
                       (hipStream_t)stream, d_tokens, rows, d_emb, V, C, d_w, d_b, eps, d_y);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_add_layer_norm(float* d_x, const float* d_delta, int64_t rows, int32_t C,
                                   const float* d_w, const float* d_b, float eps, float* d_y,
                                   void* stream) {
    HSES_REQUIRE(rows >= 0 && C >= 1, "bad sizes");
    if (rows == 0) return HSES_OK;
    HSES_REQUIRE(d_x && d_delta && d_w && d_b && d_y, "NULL pointer");
    HSES_REQUIRE(d_y != d_x && d_y != d_delta, "y must not alias x or delta");
    HSES_REQUIRE((rows + 3) / 4 < (1ll << 31), "grid too large");
    const bool al = reinterpret_cast<uintptr_t>(d_x) % 16 == 0 && reinterpret_cast<uintptr_t>(d_delta) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(d_w) % 16 == 0 && reinterpret_cast<uintptr_t>(d_b) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(d_y) % 16 == 0;
    const dim3 g(blocks_of(rows, 4)), blk(256);
    hipStream_t s = (hipStream_t)stream;
    if (al && C == 256)
        hipLaunchKernelGGL(k_add_layer_norm4<1>, g, blk, 0, s, d_x, d_delta, rows, d_w, d_b, eps, d_y);
    else if (al && C == 512)
        hipLaunchKernelGGL(k_add_layer_norm4<2>, g, blk, 0, s, d_x, d_delta, rows, d_w, d_b, eps, d_y);
    else if (al && C == 1024)
        hipLaunchKernelGGL(k_add_layer_norm4<4>, g, blk, 0, s, d_x, d_delta, rows, d_w, d_b, eps, d_y);
    else
        hipLaunchKernelGGL(k_add_layer_norm, g, blk, 0, s, d_x, d_delta, rows, C, d_w, d_b, eps, d_y);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_add_ln_shift(float* d_x, const float* d_delta, int64_t nseq, int32_t T, int32_t C,
                                 const float* d_w, const float* d_b, float eps, const float* d_state,
                                 const uint8_t* d_new_starts, const float* d_mix, int32_t n_mix,
                                 void* d_out, int32_t out_fmt, float* d_y_last, int32_t length,
                                 void* stream) {
    HSES_REQUIRE(nseq >= 0 && T >= 1 && C >= 1, "bad sizes");
    HSES_REQUIRE(out_fmt == HSES_FMT_F32 || out_fmt == HSES_FMT_BF16, "out_fmt must be F32 or BF16");
    HSES_REQUIRE(!d_y_last || (length >= 1 && length <= T), "length must be in [1, T]");
    if (nseq == 0) return HSES_OK;
    HSES_REQUIRE(d_x && d_w && d_b && d_state && d_mix && d_out, "NULL pointer");
    const auto a16 = [](const void* p) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    if (!((C == 256 || C == 512 || C == 1024) && (n_mix == 1 || n_mix == 6) && a16(d_x) && a16(d_delta) &&
          a16(d_w) && a16(d_b) && a16(d_state) && a16(d_mix) && a16(d_out) && a16(d_y_last)))
        return set_error(HSES_ERR_UNSUPPORTED,
                         "fused add + LayerNorm + token shift: C in {256, 512, 1024}, 1 or 6 mixes, "
                         "16-byte aligned buffers");
    HSES_REQUIRE((nseq + 3) / 4 < (1ll << 31), "grid too large");
    const dim3 g(blocks_of(nseq, 4)), blk(256);
    hipStream_t s = (hipStream_t)stream;
    const bool add = d_delta != nullptr, bf = out_fmt == HSES_FMT_BF16;
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, g, blk, 0, s, d_x, d_delta, nseq, T, d_w, d_b, eps, d_state,
                           d_new_starts, d_mix, d_out, d_y_last, length);
    };
    auto by_fmt = [&](auto nv, auto nm, auto ad) {
        constexpr int NV = decltype(nv)::value, NM = decltype(nm)::value;
        constexpr bool AD = decltype(ad)::value;
        if (bf) go(k_ln_shift<NV, NM, AD, true>);
        else go(k_ln_shift<NV, NM, AD, false>);
    };
    auto by_add = [&](auto nv, auto nm) {
        if (add) by_fmt(nv, nm, std::true_type{});
        else by_fmt(nv, nm, std::false_type{});
    };
    auto by_mix = [&](auto nv) {
        if (n_mix == 1) by_add(nv, std::integral_constant<int, 1>{});
        else by_add(nv, std::integral_constant<int, 6>{});
    };
    if (C == 256) by_mix(std::integral_constant<int, 1>{});
    else if (C == 512) by_mix(std::integral_constant<int, 2>{});
    else by_mix(std::integral_constant<int, 4>{});
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_tm_gates_kk(float* d_w2o, const float* d_a2o, const float* d_v2o, float* d_v,
                                const float* d_v_first, const float* d_w0, const float* d_a0,
                                const float* d_v0, float* d_k, const float* d_k_k,
                                const float* d_k_a, int64_t rows, int32_t H, int32_t S,
                                float* d_ai, float* d_bi, void* stream) {
    HSES_REQUIRE(rows >= 0 && H >= 1 && S >= 1 && S <= 64, "bad sizes (S <= 64)");
    if (rows == 0) return HSES_OK;
    HSES_REQUIRE(d_w2o && d_a2o && d_w0 && d_a0 && d_k && d_k_k && d_k_a && d_ai && d_bi,
                 "NULL pointer");
    HSES_REQUIRE(!d_v2o || (d_v && d_v_first && d_v0), "NULL pointer (v branch)");
    HSES_REQUIRE((rows * H + 3) / 4 < (1ll << 31), "grid too large");
    hipLaunchKernelGGL(k_tm_gates_kk, dim3(blocks_of(rows * H, 4)), dim3(256), 0,
                       (hipStream_t)stream, d_w2o, d_a2o, d_v2o, d_v, d_v_first, d_w0, d_a0, d_v0,
                       d_k, d_k_k, d_k_a, rows, H, S, d_ai, d_bi);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_tm_fused(const float* d_r, const float* d_w2o, const float* d_k,
                             const float* d_v, const float* d_a2o, const float* d_v2o,
                             const float* d_v_first, const float* d_w0, const float* d_a0,
                             const float* d_v0, const float* d_k_k, const float* d_k_a,
                             const float* d_s_in, const uint8_t* d_new_starts, int64_t nseq,
                             int32_t T, int32_t H, int32_t S, int32_t length, const float* d_g,
                             const float* d_ln_w, const float* d_ln_b, float eps,
                             const float* d_r_k, void* d_out, int32_t out_fmt, float* d_s_out,
                             void* stream) {
    HSES_REQUIRE(nseq >= 0 && T >= 1 && H >= 1, "bad sizes");
    HSES_REQUIRE(S == 16 || S == 32 || S == 64, "head size S must be 16, 32 or 64");
    HSES_REQUIRE(length >= 0 && length <= T, "length must be in [0, T]");
    HSES_REQUIRE(out_fmt == HSES_FMT_F32 || out_fmt == HSES_FMT_BF16, "out_fmt must be F32 or BF16");
    if (nseq == 0) return HSES_OK;
    HSES_REQUIRE(d_r && d_w2o && d_k && d_v && d_a2o && d_w0 && d_a0 && d_k_k && d_k_a &&
                     d_out && d_g && d_ln_w && d_ln_b && d_r_k,
                 "NULL pointer");
    HSES_REQUIRE(!d_v2o || (d_v_first && d_v0), "NULL pointer (value branch)");
    HSES_REQUIRE(!d_s_out || d_s_out != d_s_in, "s_out must not alias s_in");
    // Other waves still read these planes while a wave stores its output rows
    // (a bf16 out would also write 2-byte halves into fp32 rows).
    HSES_REQUIRE(d_out != d_r && d_out != d_k && d_out != d_v && d_out != d_w2o &&
                     d_out != d_a2o && d_out != d_v2o && d_out != d_v_first && d_out != d_g,
                 "out must not alias r, w, k, v, a, the value-branch inputs or g");
    return launch_wkv7<true, true>(
        d_r, d_w2o, d_k, d_v, d_a2o, nullptr, d_s_in, d_new_starts, nseq, T, H, S, length,
        static_cast<float*>(d_out), d_s_out,
        WkvPost{d_g, d_ln_w, d_ln_b, d_r_k, eps, out_fmt == HSES_FMT_BF16}, stream,
        WkvGates{d_v2o, d_v_first, d_w0, d_a0, d_v0, d_k_k, d_k_a});
}
