// linear_mw.hip -- member weights: the perturbed forward as y = x W_m^T.
//
// Reference: lora_linear_batched (burn_impl/hyperscalees-models/src/snn.rs:665-685),
// do_mm_impl (burn_impl/hyperscalees-noiser/src/eggroll.rs:419-446):
//   y_m = x W^T + sign_m (sigma / sqrt(r)) (x B_m) A_m^T,
// members 2p and 2p+1 sharing the pair's B_p and A_p with opposite signs
// (eggroll.rs:60-65).
//
// With many rows per member (an SNN member's samples x time steps: 1024 at
// C3) against the rank, forming each member's weights once is cheaper than
// the factored product: W_m = W + sign_m A'_p B_p^T (A'_p = A_p sigma / sqrt(r);
// a x b x r multiply-adds per pair, both members from one product), then
// y = x W_m^T (R x b x a per member) replaces x [W^T | B_p] (R x b x (a + r))
// and (x B_p) A_p^T (R x r x a).  At C3 (R = 1024, a = r = 128) that halves
// the matrix-core work of the forward and removes its second product.
//   k_member_weights     one workgroup per pair, a wave per 32 rows of W:
//                        the wave's rows of A'_p as MFMA operands in
//                        registers, B_p from the factor record in chunks of 32
//                        inputs, the product added to W (subtracted for the
//                        odd member) and stored as bf16 or, for the
//                        fp32-accurate mode, as the fp16 high and low parts of
//                        1024 W_m (the split form k_pair_bits<.., X> reads).
//   k_pair_bits<.., MW>  the hidden-layer kernel on those weights
//                        (pair_bits.h): each block's member's W tiles stream
//                        into LDS; no B columns, no A block, no rank product.
#include "pair_bits.h"

namespace hses {

constexpr int MW_THREADS = 256;  // 4 waves: 32 rows of W each (a <= 128)
constexpr int MW_KC = 64;        // inputs (columns of W_m) per chunk
constexpr int MW_BP = K2_NMAX + 8;  // LDS pitch of a staged B row (fp16; 272 B)

// Elements of one member's weights: (a, kp) once (bf16) or twice (high then
// low part, fp16).
static int64_t member_stride(int32_t a, int32_t b, bool split) {
    return (split ? 2 : 1) * (int64_t)a * ((b + 63) / 64 * 64);
}

// Member weights of every pair of members [tid_lo, tid_lo + n) from their
// factor record (stream rows [0, b) B, [b, a + b) A; do_mm).  One workgroup
// per pair; the product A'_p B_p^T (A' = bs A) runs over chunks of 64
// inputs:
//   * the chunk's B rows (r rank rows x 64 inputs of the record, 16-byte
//     coalesced loads, the next chunk's issued before this one's products)
//     go through LDS transposed to [input][rank] as fp16 high and low parts;
//   * wave w holds rows 32w.. of A' (times K3_XSCALE) as high and low MFMA
//     operands in registers for the whole pair and computes two 32x32 tiles
//     per chunk over K = r: A operand lane l = A'[32w + l % 32][16 s +
//     8 (l / 32) + i], B operand lane l = B[k0 + l % 32][16 s + 8 (l / 32) +
//     i], result lane l = rows 32w + 8 g + 4 (l / 32) + v of column k0 + l % 32;
//     three products (hi hi, hi lo, lo hi) give 1024 A'_p B_p^T to fp32
//     accuracy;
//   * the wave's 32 x 64 result goes through its own LDS scratch so that each
//     lane then owns runs of 8 consecutive inputs of one row: W is read and
//     the results stored with 16-byte accesses.  X: 1024 W (exact) +- the
//     product, split again into high and low parts; else W +- 2^-10 of it,
//     rounded once to bf16.
constexpr int MW_SP = MW_KC + 4;  // scratch pitch (floats)
template <bool X>
__global__ __launch_bounds__(MW_THREADS, 2) void k_member_weights(
    const float* __restrict__ W, const float* __restrict__ rec, int32_t a, int32_t b, int32_t r,
    float bs, int32_t tid_lo, int32_t n, int32_t pair_lo, uint16_t* __restrict__ wm,
    int64_t wm_stride) {
    // [hi, lo][k][c] B chunk (2 x 64 x 136 fp16), then per wave a 32 x 68
    // fp32 scratch (69.6 KB, dynamic)
    extern __shared__ __align__(16) uint16_t mw_lds[];
    uint16_t* Bh = mw_lds;
    uint16_t* Bl = mw_lds + MW_KC * MW_BP;
    const int32_t pi = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    float* scr = reinterpret_cast<float*>(mw_lds + 2 * MW_KC * MW_BP) + wave * 32 * MW_SP;
    const int lc = lane & 31, hl = lane >> 5;
    const int32_t o0 = 32 * wave;
    const int32_t kp = (b + 63) / 64 * 64, ab = a + b;
    const float* rp = rec + (size_t)pi * r * ab;
    const int32_t m_even = 2 * (pair_lo + pi) - tid_lo;  // -1: the pair's even member is absent
    const bool has_even = m_even >= 0, has_odd = m_even + 1 < n;
    const int64_t off_even = (int64_t)m_even * wm_stride, off_odd = off_even + wm_stride;
    const int64_t lo_off = (int64_t)a * kp;  // X: the low part after the high part
    const bool wave_on = o0 < a;             // waves past a stage B but compute nothing

    // this wave's rows of A' (rows past a repeat row a - 1; never stored)
    const int32_t oa = min(o0 + lc, a - 1);
    u16x8 ah[8], al[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        ah[s] = u16x8{};
        al[s] = u16x8{};
        if (wave_on && 16 * s < r) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                // (normal * bs) rounded once, as the forward scales it; the
                // power-of-two K3_XSCALE after that is exact
                uint16_t h, l;
                split_f16(rp[(size_t)(16 * s + 8 * hl + i) * ab + b + oa] * bs * K3_XSCALE, &h, &l);
                ah[s][i] = h;
                al[s][i] = l;
            }
        }
    }

    // B staging: thread t loads rank row c = t / 2, inputs k0 + 32 (t % 2) +
    // [0, 32) as 8 float4 (zero past b or past r)
    const int32_t sc = tid >> 1, sk = (tid & 1) * 32;
    // 16-byte loads when every record row starts 16-byte aligned
    const bool vec = ((uintptr_t)rec % 16 == 0) && (ab % 4 == 0);
    float4 bv[8];
    auto bload = [&](int32_t k0) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int32_t k = k0 + sk + 4 * q;
            if (vec && sc < r && k + 3 < b) {
                bv[q] = *reinterpret_cast<const float4*>(rp + (size_t)sc * ab + k);
            } else {
                float e[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) e[u] = (sc < r && k + u < b) ? rp[(size_t)sc * ab + k + u] : 0.0f;
                bv[q] = make_float4(e[0], e[1], e[2], e[3]);
            }
        }
    };
    auto bstore = [&]() {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float e[4] = {bv[q].x, bv[q].y, bv[q].z, bv[q].w};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                uint16_t h, l;
                split_f16(e[u], &h, &l);
                const int32_t at = (sk + 4 * q + u) * MW_BP + sc;
                Bh[at] = h;
                Bl[at] = l;
            }
        }
    };
    // W rows 16-byte aligned: 8 consecutive inputs as two float4
    const bool wvec = ((uintptr_t)W % 16 == 0) && (b % 4 == 0);
    const int32_t nch = kp / MW_KC;
    bload(0);
    bstore();
    __syncthreads();
    for (int32_t ch = 0; ch < nch; ++ch) {
        const int32_t k0 = ch * MW_KC;
        if (ch + 1 < nch) bload(k0 + MW_KC);
        f32x16 acc[2] = {f32x16{}, f32x16{}};
        if (wave_on) {
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                if (16 * s >= r) break;
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const int32_t at = (32 * t + lc) * MW_BP + 16 * s + 8 * hl;
                    const u16x8 bh = *reinterpret_cast<const u16x8*>(Bh + at);
                    const u16x8 bl = *reinterpret_cast<const u16x8*>(Bl + at);
                    acc[t] = mfma32_f16(ah[s], bh, acc[t]);
                    acc[t] = mfma32_f16(ah[s], bl, acc[t]);
                    acc[t] = mfma32_f16(al[s], bh, acc[t]);
                }
            }
        }
        __syncthreads();  // every wave has read this chunk's B
        if (ch + 1 < nch) bstore();
        if (wave_on) {
            // result -> the wave's scratch [row][input]
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    scr[(8 * (v >> 2) + 4 * hl + (v & 3)) * MW_SP + 32 * t + lc] = acc[t][v];
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
            // lane: runs (row, 8 inputs) number lane + 64 q of the 32 x 8
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int32_t run = lane + 64 * q, row = run >> 3, k8 = (run & 7) * 8;
                const int32_t o = o0 + row, k = k0 + k8;
                if (o >= a) continue;
                float p[8], w[8];
                *reinterpret_cast<float4*>(p) = *reinterpret_cast<const float4*>(scr + row * MW_SP + k8);
                *reinterpret_cast<float4*>(p + 4) =
                    *reinterpret_cast<const float4*>(scr + row * MW_SP + k8 + 4);
                const float* wr = W + (size_t)o * b + k;
                if (wvec && k + 7 < b) {
                    *reinterpret_cast<float4*>(w) = *reinterpret_cast<const float4*>(wr);
                    *reinterpret_cast<float4*>(w + 4) = *reinterpret_cast<const float4*>(wr + 4);
                } else {
#pragma unroll
                    for (int u = 0; u < 8; ++u) w[u] = k + u < b ? wr[u] : 0.0f;
                }
                const int64_t at = (int64_t)o * kp + k;
                if constexpr (X) {
                    u16x8 eh, el, oh, ol;
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const float base = w[u] * K3_XSCALE;  // exact
                        uint16_t h, l;
                        split_f16(base + p[u], &h, &l);
                        eh[u] = h;
                        el[u] = l;
                        split_f16(base - p[u], &h, &l);
                        oh[u] = h;
                        ol[u] = l;
                    }
                    if (has_even) {
                        *reinterpret_cast<u16x8*>(wm + off_even + at) = eh;
                        *reinterpret_cast<u16x8*>(wm + off_even + lo_off + at) = el;
                    }
                    if (has_odd) {
                        *reinterpret_cast<u16x8*>(wm + off_odd + at) = oh;
                        *reinterpret_cast<u16x8*>(wm + off_odd + lo_off + at) = ol;
                    }
                } else {
                    u16x8 e, od;
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const float d = p[u] * (1.0f / K3_XSCALE);  // exact
                        e[u] = f2bf(w[u] + d);
                        od[u] = f2bf(w[u] - d);
                    }
                    if (has_even) *reinterpret_cast<u16x8*>(wm + off_even + at) = e;
                    if (has_odd) *reinterpret_cast<u16x8*>(wm + off_odd + at) = od;
                }
            }
        }
        __syncthreads();  // the next chunk's B is in LDS
    }
}

size_t member_weights_bytes(int32_t a, int32_t b, int32_t n, bool split) {
    if (a < 1 || b < 1 || n < 1) return 0;
    return (size_t)n * member_stride(a, b, split) * 2;
}

int launch_member_weights(const float* W, const float* rec, int32_t a, int32_t b, int32_t r,
                          float bs, int32_t tid_lo, int32_t n, bool split, uint16_t* wm,
                          hipStream_t s) {
    if (a > K2_NMAX || r < 16 || r > K2_NMAX || r % 16) return HSES_ERR_UNSUPPORTED;
    int32_t lo, cnt;
    pair_range(tid_lo, n, &lo, &cnt);
    const int64_t stride = member_stride(a, b, split);
    const size_t lds = (size_t)2 * MW_KC * MW_BP * 2 + (size_t)(MW_THREADS / 64) * 32 * MW_SP * 4;
    auto launch = [&](auto kern) -> int {
        HSES_CHECK_HIP(hipFuncSetAttribute((const void*)kern,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        hipLaunchKernelGGL(kern, dim3((uint32_t)cnt), dim3(MW_THREADS), lds, s, W, rec, a, b, r,
                           bs, tid_lo, n, lo, wm, stride);
        return HSES_OK;
    };
    int rc = split ? launch(k_member_weights<true>) : launch(k_member_weights<false>);
    if (rc) return rc;
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

// The forward on member weights: k_pair_bits<.., MW> over members
// [tid_lo, tid_lo + n), bit-packed x, rows per member a multiple of K3_RB.
int launch_linear_mw(LinParams& P, DeviceState* st, hipStream_t s, const LifOut* lif) {
    const bool xm = P.math == HSES_MATH_F32X;
    if (P.x_fmt != HSES_FMT_BITS || P.a > K2_NMAX || P.R % K3_RB || P.b > 2 * K3_XPF * 64 ||
        P.tmm)
        return HSES_ERR_UNSUPPORTED;
    // the two-buffer stream needs two stream tiles per block: K of more than
    // one tile, or the split form (each K tile streamed twice)
    if (!xm && P.b <= 64) return HSES_ERR_UNSUPPORTED;
    if (lif && (P.n_time > 16 || (P.n_time & (P.n_time - 1)) != 0)) return HSES_ERR_UNSUPPORTED;
    const K3Layout lay(P.r, P.b, true, xm, true);
    if (lay.bytes > st->max_lds) return HSES_ERR_UNSUPPORTED;
    K2Args A{};
    pair_range(P.tid_lo, P.n, &A.pair_lo, &A.n_pairs);
    int32_t grid = pair_grid(st, A.n_pairs);
    // pairs split over 4 workgroups of one XCD, as in launch_linear_pair: the
    // member's weights are fetched about once and re-read from that XCD's L2
    A.split = 1;
    if (P.tid_lo % 2 == 0 && P.n % 2 == 0 && (2 * (int64_t)P.R) % (4 * K3_RB) == 0 &&
        st->num_cus % 32 == 0 && (int64_t)A.n_pairs * 4 >= st->num_cus) {
        A.split = 4;
        grid = st->num_cus;
    }
    A.group = 1;
    A.x = P.x;
    A.x_stride = P.x_stride;
    A.x_plane = P.x_plane;
    A.y = P.y;
    A.y_stride = P.y_stride;
    A.y_plane = P.y_plane;
    A.a = P.a;
    A.b = P.b;
    A.r = P.r;
    A.R = P.R;
    A.rpm = P.rpm;
    A.T = P.n_time;
    if (lif) {
        A.spk = static_cast<uint64_t*>(lif->spk);
        A.spk_stride = lif->spk_stride;
        A.spk_plane = lif->spk_plane;
        A.rate = lif->rate;
        A.rate_stride = lif->rate_stride;
        A.cpl = static_cast<uint64_t*>(lif->cpl);
        A.cpl_stride = lif->cpl_stride;
        A.leak = lif->leak;
        A.v_th = lif->v_th;
    }
    A.n = P.n;
    A.tid_lo = P.tid_lo;
    A.wm = P.wm;
    A.wm_stride = P.wm_stride;
    {
        const int64_t words = (P.b + 63) / 64;
        A.x_vec = 0;
        A.x_packed = reinterpret_cast<uintptr_t>(P.x) % 16 == 0 && P.x_plane == words &&
                     P.x_stride == (int64_t)P.n_time * words && ((int64_t)P.R * words) % 2 == 0;
    }
    auto launch = [&](auto kern) -> int {
        if (lay.bytes > 64 * 1024)
            HSES_CHECK_HIP(hipFuncSetAttribute((const void*)kern,
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)lay.bytes));
        hipLaunchKernelGGL(kern, dim3(grid), dim3(K3_THREADS), lay.bytes, s, A);
        HSES_CHECK_HIP(hipGetLastError());
        return HSES_OK;
    };
    auto by_math = [&](auto xc) -> int {
        constexpr bool XX = decltype(xc)::value;
        if (!lif) {
            if (P.a <= 32) return launch(k_pair_bits<EPI_Y, 1, false, false, true, true, XX, 1, true>);
            return launch(k_pair_bits<EPI_Y, 1, false, false, true, true, XX, 4, true>);
        }
        const bool spk = lif->spk != nullptr, rate = lif->rate != nullptr || lif->cpl != nullptr;
        auto by_t = [&](auto sc, auto rc) -> int {
            constexpr bool S = decltype(sc)::value, Q = decltype(rc)::value;
            switch (P.n_time) {
                case 1: return launch(k_pair_bits<EPI_LIF, 1, S, Q, true, true, XX, 4, true>);
                case 2: return launch(k_pair_bits<EPI_LIF, 2, S, Q, true, true, XX, 4, true>);
                case 4: return launch(k_pair_bits<EPI_LIF, 4, S, Q, true, true, XX, 4, true>);
                case 8: return launch(k_pair_bits<EPI_LIF, 8, S, Q, true, true, XX, 4, true>);
                default: return launch(k_pair_bits<EPI_LIF, 16, S, Q, true, true, XX, 4, true>);
            }
        };
        if (spk && rate) return by_t(std::true_type{}, std::true_type{});
        if (spk) return by_t(std::true_type{}, std::false_type{});
        return by_t(std::false_type{}, std::true_type{});
    };
    return xm ? by_math(std::true_type{}) : by_math(std::false_type{});
}

}  // namespace hses
