// linear.hip -- batched EggRoll perturbed forward  y = x W^T + (x B_m) A_m^T.
//
// Reference: do_mm_impl (burn_impl/hyperscalees-noiser/src/eggroll.rs:419-446)
// and its batched form lora_linear_batched (burn_impl/hyperscalees-models/src/snn.rs:665-685).
//
// k_linear_small (this file) serves ranks whose noise columns fit beside a
// 64-wide output tile (members_per_tile * r <= 64): C1 (r=4), C2 (r=1).
// A workgroup owns 64 consecutive member-major rows and 64 output columns:
//   1. generates B_m (all K rows) and the tile's rows of A_m for the members
//      its rows belong to, straight into LDS (never to HBM);
//   2. runs the K loop with MFMA over [W_tile^T | B_m...] (x tile and W tile
//      staged through LDS, B_m resident), giving x W^T and x B_m together;
//   3. adds (x B_m) A_m^T in the epilogue (r multiply-adds per output).
// Larger ranks go to k_linear_pair (linear_pair.hip).
#include <math.h>

#include "linear_common.h"
#include "mfma.h"
#include "noise_dev.h"
#include "runtime.h"
#include "tile_factors.h"

namespace hses {

constexpr int K1_BM = 64, K1_CT = 64, K1_BK = 32, K1_THREADS = 256, K1_NEMAX = 64;

template <int MATH>
struct K1Layout {
    using T = typename MathT<MATH>::T;
    static constexpr int PAD = MathT<MATH>::PAD;
    static constexpr int XP = K1_BK + PAD;  // pitch of the x and W tiles
    size_t off_x, off_w, off_b, off_a, off_xb, bytes;
    __host__ __device__ K1Layout(int ne_real, int ne, int bpitch, int nm_max, int r) {
        size_t o = align16(sizeof(BmTables));
        off_x = o;
        o = align16(o + (size_t)K1_BM * XP * sizeof(T));
        off_w = o;
        o = align16(o + (size_t)K1_CT * XP * sizeof(T));
        off_b = o;
        o = align16(o + (size_t)ne_real * bpitch * sizeof(T));
        off_a = o;
        o = align16(o + (size_t)nm_max * K1_CT * r * sizeof(float));
        off_xb = o;
        o = align16(o + (size_t)K1_BM * ne * sizeof(float));
        bytes = o;
    }
};

template <int MATH, int XFMT>
__global__ __launch_bounds__(K1_THREADS) void k_linear_small(LinParams P) {
    using T = typename MathT<MATH>::T;
    using L = K1Layout<MATH>;
    constexpr int XP = L::XP;
    extern __shared__ __align__(16) unsigned char smem[];
    const L lay(P.ne_real, P.ne, P.bpitch, P.nm_max, P.r);
    BmTables* tabs = reinterpret_cast<BmTables*>(smem);
    T* Xs = reinterpret_cast<T*>(smem + lay.off_x);
    T* Ws = reinterpret_cast<T*>(smem + lay.off_w);
    T* Bs = reinterpret_cast<T*>(smem + lay.off_b);
    float* As = reinterpret_cast<float*>(smem + lay.off_a);
    float* XB = reinterpret_cast<float*>(smem + lay.off_xb);

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int64_t L0 = (int64_t)blockIdx.x * K1_BM;
    const int32_t o0 = blockIdx.y * K1_CT;
    const int32_t ct = min(K1_CT, P.a - o0);
    const int32_t R = P.R, r = P.r, b = P.b;
    const int32_t m_first = (int32_t)(L0 / R);
    const int32_t m_last = (int32_t)((min(L0 + K1_BM, P.total) - 1) / R);
    const int32_t nm = m_last - m_first + 1;
    const bool noisy = P.ne > 0;

    // ---- 1. factors of the tile's members into LDS -------------------------
    if (noisy) {
        load_bm_tables(tabs, P.tables);
        for (int i = tid; i < P.ne_real * P.bpitch; i += K1_THREADS) Bs[i] = MathT<MATH>::zero();
        __syncthreads();
        const NoiseCtx ctx{tabs, P.log_exc, P.cos_exc};
        gen_tile_factors<MATH>(P, ctx, m_first, nm, o0, ct, Bs, P.bpitch, As, K1_CT);
    }
    __syncthreads();

    // ---- 2. K loop ----------------------------------------------------------
    f32x4 accb[K1_CT / 16], accx[K1_NEMAX / 16];
#pragma unroll
    for (int i = 0; i < K1_CT / 16; ++i) accb[i] = f32x4{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < K1_NEMAX / 16; ++i) accx[i] = f32x4{0, 0, 0, 0};
    const int ne_tiles = P.ne / 16;
    const int srow = tid >> 2, sk = (tid & 3) * 8;  // staging: 64 rows x 4 segments of 8
    const int64_t Lrow = L0 + srow;
    const bool rvalid = Lrow < P.total;
    const int64_t xoff = rvalid ? phys_row(P, Lrow, P.x_stride, P.x_plane) : 0;
    const int32_t wcol = o0 + srow;
    const int mrow = wave * 16 + (lane & 15), kg = lane >> 4;

    for (int32_t k0 = 0; k0 < b; k0 += K1_BK) {
        T xv[8], wv[8];
        load_x_seg<MATH, XFMT>(P.x, xoff, rvalid, k0 + sk, b, xv);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int32_t k = k0 + sk + i;
            const int64_t wi = P.tmm ? (int64_t)k * P.a + wcol : (int64_t)wcol * b + k;
            wv[i] = MathT<MATH>::cvt((wcol < P.a && k < b) ? P.W[wi] : 0.0f);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            Xs[srow * XP + sk + i] = xv[i];
            Ws[srow * XP + sk + i] = wv[i];
        }
        __syncthreads();
        if constexpr (MATH == HSES_MATH_F32) {
#pragma unroll
            for (int ks = 0; ks < K1_BK; ks += 4) {
                const float af = Xs[mrow * XP + ks + kg];
#pragma unroll
                for (int nt = 0; nt < K1_CT / 16; ++nt)
                    if (nt * 16 < ct) accb[nt] = mfma_f32(af, Ws[(nt * 16 + (lane & 15)) * XP + ks + kg], accb[nt]);
#pragma unroll
                for (int ne = 0; ne < K1_NEMAX / 16; ++ne)
                    if (ne < ne_tiles) {
                        const int br = ne * 16 + (lane & 15);
                        const float bf = br < P.ne_real ? Bs[(size_t)br * P.bpitch + k0 + ks + kg] : 0.0f;
                        accx[ne] = mfma_f32(af, bf, accx[ne]);
                    }
            }
        } else {
            const u16x8 af = lds_u16x8(&Xs[mrow * XP + kg * 8]);
#pragma unroll
            for (int nt = 0; nt < K1_CT / 16; ++nt)
                if (nt * 16 < ct) accb[nt] = mfma_bf16(af, lds_u16x8(&Ws[(nt * 16 + (lane & 15)) * XP + kg * 8]), accb[nt]);
#pragma unroll
            for (int ne = 0; ne < K1_NEMAX / 16; ++ne)
                if (ne < ne_tiles) {
                    const int br = ne * 16 + (lane & 15);
                    const u16x8 bf = br < P.ne_real ? lds_u16x8(&Bs[(size_t)br * P.bpitch + k0 + kg * 8])
                                                    : u16x8{0, 0, 0, 0, 0, 0, 0, 0};
                    accx[ne] = mfma_bf16(af, bf, accx[ne]);
                }
        }
        __syncthreads();
    }

    // ---- 3. epilogue: y = x W^T + (x B_m) A_m^T ------------------------------
    if (noisy) {
#pragma unroll
        for (int ne = 0; ne < K1_NEMAX / 16; ++ne)
            if (ne < ne_tiles) {
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    XB[(wave * 16 + 4 * kg + v) * P.ne + ne * 16 + (lane & 15)] = accx[ne][v];
            }
        __syncthreads();
    }
#pragma unroll
    for (int nt = 0; nt < K1_CT / 16; ++nt) {
        const int col = nt * 16 + (lane & 15);
        if (nt * 16 >= ct || col >= ct) continue;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int row = wave * 16 + 4 * kg + v;
            const int64_t Lr = L0 + row;
            if (Lr >= P.total) continue;
            float yv = accb[nt][v];
            if (noisy) {
                const int32_t lm = (int32_t)(Lr / R) - m_first;
                const float* xb = XB + row * P.ne + lm * r;
                const float* ar = As + ((size_t)lm * K1_CT + col) * r;
                float z = 0.0f;
                for (int32_t c = 0; c < r; ++c) z = __fadd_rn(z, __fmul_rn(xb[c], ar[c]));
                yv = __fadd_rn(yv, z);
            }
            P.y[phys_row(P, Lr, P.y_stride, P.y_plane) + o0 + col] = yv;
        }
    }
}

template <int MATH>
static size_t k1_lds_bytes(const LinParams& P) {
    return K1Layout<MATH>(P.ne_real, P.ne, P.bpitch, P.nm_max, P.r).bytes;
}

template <int MATH, int XFMT>
static int launch_small(const LinParams& P, size_t lds, hipStream_t s) {
    auto kern = k_linear_small<MATH, XFMT>;
    if (lds > 64 * 1024)
        HSES_CHECK_HIP(hipFuncSetAttribute((const void*)kern,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    const int64_t row_tiles = (P.total + K1_BM - 1) / K1_BM;
    const int col_tiles = (P.a + K1_CT - 1) / K1_CT;
    hipLaunchKernelGGL(kern, dim3((uint32_t)row_tiles, col_tiles), dim3(K1_THREADS), lds, s, P);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

int launch_linear_small(LinParams& P, DeviceState* st, hipStream_t s) {
    // Members a 64-row tile can touch.
    int32_t nm_max;
    if (P.R % K1_BM == 0)
        nm_max = 1;
    else if (K1_BM % P.R == 0)
        nm_max = K1_BM / P.R;
    else
        nm_max = (K1_BM - 1) / P.R + 2;
    nm_max = std::min(nm_max, P.n);
    const bool noisy = P.r > 0 && P.bs != 0.0f;
    P.nm_max = nm_max;
    P.ne_real = noisy ? nm_max * P.r : 0;
    P.ne = (P.ne_real + 15) / 16 * 16;
    if (P.ne > K1_NEMAX) return HSES_ERR_UNSUPPORTED;
    P.rc = noisy ? std::max(1, 32 / P.r) : 1;
    P.bpitch = (P.b + K1_BK - 1) / K1_BK * K1_BK + (P.math == HSES_MATH_F32 ? 4 : 8);
    const size_t lds = P.math == HSES_MATH_F32 ? k1_lds_bytes<HSES_MATH_F32>(P)
                                               : k1_lds_bytes<HSES_MATH_BF16>(P);
    if (lds > st->max_lds) return HSES_ERR_UNSUPPORTED;
    if (noisy) {
        const int64_t chunks = (P.a + P.b + P.rc - 1) / P.rc;
        int rc = get_jump_table(st, (int64_t)P.rc * P.r, chunks, &P.jump);
        if (rc) return rc;
    }
    const int key = P.math * 4 + P.x_fmt;
    switch (key) {
        case HSES_MATH_F32 * 4 + HSES_FMT_F32: return launch_small<HSES_MATH_F32, HSES_FMT_F32>(P, lds, s);
        case HSES_MATH_F32 * 4 + HSES_FMT_BF16: return launch_small<HSES_MATH_F32, HSES_FMT_BF16>(P, lds, s);
        case HSES_MATH_F32 * 4 + HSES_FMT_BITS: return launch_small<HSES_MATH_F32, HSES_FMT_BITS>(P, lds, s);
        case HSES_MATH_BF16 * 4 + HSES_FMT_F32: return launch_small<HSES_MATH_BF16, HSES_FMT_F32>(P, lds, s);
        case HSES_MATH_BF16 * 4 + HSES_FMT_BF16: return launch_small<HSES_MATH_BF16, HSES_FMT_BF16>(P, lds, s);
        case HSES_MATH_BF16 * 4 + HSES_FMT_BITS: return launch_small<HSES_MATH_BF16, HSES_FMT_BITS>(P, lds, s);
        default: return set_error(HSES_ERR_INVALID_ARG, "unsupported x format");
    }
}

}  // namespace hses

using namespace hses;

extern "C" size_t hses_perturbed_linear_workspace(int32_t a, int32_t b, int32_t rank, int32_t n,
                                                  int32_t rows_per_member, int32_t n_time,
                                                  int32_t math) {
    if (math == HSES_MATH_F32)  // the fp32 GEMM's factor rows (k_linear_small needs none)
        return linear_f32_workspace(a, b, rank, n, rows_per_member, n_time, math);
    if (a < 1 || b < 1 || n < 1 || rank < 16 || rank % 16 || rank > 128 || a > 128 ||
        (math != HSES_MATH_BF16 && math != HSES_MATH_F32X))
        // the bf16 GEMM (bf16 W, factor rows), the wide-output kernel (bf16 W) or
        // k_linear_small (no workspace)
        return std::max(linear_bf16_workspace(a, b, rank, n, rows_per_member, n_time, math),
                        linear_wide_workspace(a, b, rank, n, rows_per_member, n_time, math));
    DeviceState* st;
    if (get_state(&st)) return 0;
    return linear_pair_workspace(st, a, b, rank, n);
}

// Validation and parameter block shared by the two forward entry points.
static int make_params(LinParams* P, const void* d_x, int32_t x_fmt, int64_t x_stride,
                       int64_t x_plane, int32_t n_time, const float* d_W, int32_t a, int32_t b,
                       uint64_t key, int32_t rank, float sigma, int32_t epoch, int32_t noise_reuse,
                       int32_t tid_lo, int32_t n, int32_t rows_per_member, int32_t math,
                       DeviceState** st) {
    HSES_REQUIRE(x_fmt == HSES_FMT_F32 || x_fmt == HSES_FMT_BF16 || x_fmt == HSES_FMT_BITS,
                 "x_fmt must be F32, BF16 or BITS");
    HSES_REQUIRE(math == HSES_MATH_F32 || math == HSES_MATH_BF16, "unknown math mode");
    HSES_REQUIRE(a >= 1 && b >= 1, "a and b must be >= 1");
    HSES_REQUIRE(n >= 0 && rank >= 0 && n_time >= 1 && rows_per_member >= 1, "bad sizes");
    HSES_REQUIRE(noise_reuse >= 0, "noise_reuse must be >= 0");
    HSES_REQUIRE((int64_t)tid_lo + n - 1 <= INT32_MAX && tid_lo >= 0, "thread id range");
    if (n == 0) return HSES_OK;
    HSES_REQUIRE(d_x && d_W, "NULL pointer");
    const int64_t units = x_fmt == HSES_FMT_BITS ? (b + 63) / 64 : b;
    const int64_t M = (int64_t)n * rows_per_member;
    HSES_REQUIRE(rows_layout_ok(units, M, n_time, x_stride, x_plane),
                 "x rows overlap (x_stride smaller than a row, or time planes overlap)");
    HSES_REQUIRE(M * n_time < (1ll << 40), "too many rows");
    int rc = get_state(st);
    if (rc) return rc;
    *P = LinParams{};
    P->x = d_x;
    P->x_fmt = x_fmt;
    P->x_stride = x_stride;
    P->x_plane = x_plane;
    P->n_time = n_time;
    P->rpm = rows_per_member;
    P->W = d_W;
    P->a = a;
    P->b = b;
    P->key = key;
    P->r = (sigma != 0.0f) ? rank : 0;
    P->bs = rank > 0 ? sigma / sqrtf((float)rank) : 0.0f;  // eggroll.rs:433
    P->epoch = epoch;
    P->nreuse = noise_reuse;
    P->tid_lo = tid_lo;
    P->n = n;
    P->math = math;
    P->R = n_time * rows_per_member;
    P->total = (int64_t)n * P->R;
    P->tables = (*st)->d_tables;
    P->log_exc = (*st)->d_log_exc;
    P->cos_exc = (*st)->d_cos_exc;
    return HSES_OK;
}

// The activation applied in place to y when the forward kernel did not fuse it.
template <int ACT>
__global__ void k_act_rows(LinParams P) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= P.total * P.a) return;
    const int64_t L = e / P.a;
    const int32_t c = (int32_t)(e - L * P.a);
    float* y = P.y + phys_row(P, L, P.y_stride, P.y_plane) + c;
    const float v = *y;
    if constexpr (ACT == ACT_TANH) *y = tanhf(v);
    if constexpr (ACT == ACT_SIGMOID) *y = 1.0f / (1.0f + expf(-v));
    if constexpr (ACT == ACT_RELU_SQ) {
        const float z = v > 0.0f ? v : 0.0f;
        *y = z * z;
    }
}

// Few rows per member (readouts on pooled rows): one wave per member.  The
// wave generates the member's factor rows into LDS (B rows [0, b), A rows
// [b, a+b) scaled by sign * base_sigma), then per row of the member forms
// xb = x B (lanes over the rank) and y = x W^T + xb A^T (lanes over outputs),
// every sum in index order with f32 accumulation.  fp32 math, do_mm
// orientation, F32 or BF16 activations.
constexpr int KR_MAXF = 16384;  // (a + b) * r + b floats of LDS per member
__global__ __launch_bounds__(64) void k_linear_rows(LinParams P) {
    extern __shared__ float smem[];
    __shared__ BmTables tabs;
    const int lane = threadIdx.x;
    const int32_t m = blockIdx.x;
    const int32_t r = P.r, a = P.a, b = P.b;
    float* Bs = smem;                     // (b, r)
    float* As = smem + (size_t)b * r;     // (a, r)
    float* xs = As + (size_t)a * r;       // (b) current row
    float* xb = xs + b;                   // (r)
    if (r > 0) {
        load_bm_tables(&tabs, P.tables);
        __syncthreads();
        const NoiseCtx ctx{&tabs, P.log_exc, P.cos_exc};
        float sign;
        const uint64_t seed = member_seed(P.key, P.epoch, P.nreuse, P.tid_lo + m, &sign);
        const float sc = sign * P.bs;
        for (int32_t j = lane; j < a + b; j += 64) {
            uint64_t s = row_start_state(seed, j, P.jump);
            if (j < b) {
                float* dst = Bs + (size_t)j * r;
                bm_run(s, r, ctx, [&](int32_t c, float v) { dst[c] = v; });
            } else {
                float* dst = As + (size_t)(j - b) * r;
                bm_run(s, r, ctx, [&](int32_t c, float v) { dst[c] = v * sc; });
            }
        }
    }
    __syncthreads();
    for (int32_t q = 0; q < P.R; ++q) {
        const int64_t L = (int64_t)m * P.R + q;
        const int64_t xo = phys_row(P, L, P.x_stride, P.x_plane);
        for (int32_t k = lane; k < b; k += 64) {
            if (P.x_fmt == HSES_FMT_F32) {
                xs[k] = static_cast<const float*>(P.x)[xo + k];
            } else {
                const uint32_t u = static_cast<const uint16_t*>(P.x)[xo + k];
                xs[k] = __builtin_bit_cast(float, u << 16);
            }
        }
        __syncthreads();
        if (lane < r) {
            float s = 0.0f;
            for (int32_t k = 0; k < b; ++k) s = s + xs[k] * Bs[(size_t)k * r + lane];
            xb[lane] = s;
        }
        __syncthreads();
        float* y = P.y + phys_row(P, L, P.y_stride, P.y_plane);
        for (int32_t o = lane; o < a; o += 64) {
            const float* w = P.W + (size_t)o * b;
            float base = 0.0f;
            for (int32_t k = 0; k < b; ++k) base = base + xs[k] * w[k];
            float lo = 0.0f;
            for (int32_t c = 0; c < r; ++c) lo = lo + xb[c] * As[(size_t)o * r + c];
            y[o] = r > 0 ? base + lo : base;
        }
        __syncthreads();
    }
}

static int launch_linear_rows(LinParams& P, DeviceState* st, hipStream_t s) {
    if (P.math != HSES_MATH_F32 || P.tmm || P.x_fmt == HSES_FMT_BITS || P.r > 64)
        return HSES_ERR_UNSUPPORTED;
    const size_t nf = (size_t)(P.a + P.b) * P.r + P.b + 64;
    if (nf > KR_MAXF) return HSES_ERR_UNSUPPORTED;
    if (P.r > 0) {
        int rc = get_jump_table(st, P.r, (int64_t)P.a + P.b, &P.jump);
        if (rc) return rc;
    }
    const size_t lds = nf * sizeof(float);
    if (lds > 48 * 1024)
        HSES_CHECK_HIP(hipFuncSetAttribute((const void*)k_linear_rows,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipLaunchKernelGGL(k_linear_rows, dim3((uint32_t)P.n), dim3(64), lds, s, P);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

// Output checks and the kernel choice shared by do_mm and do_Tmm: the pair
// kernels (rank a multiple of 16, output width <= 128, bf16), the wide-output
// kernel (bf16, small rank), or else the small-rank kernel.
static int run_linear(LinParams& P, DeviceState* st, float* d_y, int64_t y_stride,
                      int64_t y_plane, void* d_work, size_t work_bytes, void* stream,
                      const char* name, int32_t act = ACT_NONE, int32_t y_fmt = HSES_FMT_F32) {
    HSES_REQUIRE(d_y, "NULL pointer");
    HSES_REQUIRE(rows_layout_ok(P.a, (int64_t)P.n * P.rpm, P.n_time, y_stride, y_plane),
                 "y rows overlap (y_stride smaller than a row, or time planes overlap)");
    HSES_REQUIRE(act >= ACT_NONE && act <= ACT_RELU_SQ, "unknown activation");
    P.y = d_y;
    P.y_stride = y_stride;
    P.y_plane = y_plane;
    hipStream_t s = (hipStream_t)stream;
    HSES_REQUIRE(y_fmt == HSES_FMT_F32 || y_fmt == HSES_FMT_BF16, "y_fmt must be F32 or BF16");
    int rc = y_fmt == HSES_FMT_F32 ? launch_linear_pair(P, st, s, d_work, work_bytes)
                                   : HSES_ERR_UNSUPPORTED;
    if (rc == HSES_ERR_UNSUPPORTED) {
        rc = launch_linear_bf16(P, st, s, d_work, work_bytes, act, y_fmt);
        if (rc != HSES_ERR_UNSUPPORTED) return rc;  // activation fused
        rc = launch_linear_wide(P, st, s, d_work, work_bytes, act, y_fmt);
        if (rc != HSES_ERR_UNSUPPORTED) return rc;  // activation fused
        if (y_fmt != HSES_FMT_F32)
            return set_error(HSES_ERR_UNSUPPORTED,
                             std::string(name) + ": bf16 output needs the wide-output kernel (bf16 "
                             "math, members per 128-row tile x rank <= 16, aligned x rows)");
        rc = launch_linear_f32(P, st, s, d_work, work_bytes);
        if (rc == HSES_ERR_UNSUPPORTED) rc = launch_linear_small(P, st, s);
        if (rc == HSES_ERR_UNSUPPORTED && P.R <= 16) rc = launch_linear_rows(P, st, s);
    }
    if (rc == HSES_ERR_UNSUPPORTED)
        return set_error(HSES_ERR_UNSUPPORTED,
                         std::string(name) + ": no kernel for this rank/shape (members per 64-row "
                         "tile x rank must be <= 64, or rank a multiple of 16, or at most 16 fp32 "
                         "rows per member with (a + b) x rank <= 16000)");
    if (rc || act == ACT_NONE) return rc;
    const int64_t n = P.total * P.a;
    HSES_REQUIRE((n + 255) / 256 < (1ll << 31), "grid too large");
    const dim3 g((uint32_t)((n + 255) / 256));
    switch (act) {
        case ACT_TANH: hipLaunchKernelGGL(k_act_rows<ACT_TANH>, g, dim3(256), 0, s, P); break;
        case ACT_SIGMOID: hipLaunchKernelGGL(k_act_rows<ACT_SIGMOID>, g, dim3(256), 0, s, P); break;
        default: hipLaunchKernelGGL(k_act_rows<ACT_RELU_SQ>, g, dim3(256), 0, s, P); break;
    }
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

extern "C" int hses_perturbed_linear(const void* d_x, int32_t x_fmt, int64_t x_stride,
                                     int64_t x_plane, int32_t n_time, const float* d_W, int32_t a,
                                     int32_t b, uint64_t key, int32_t rank, float sigma,
                                     int32_t epoch, int32_t noise_reuse, int32_t tid_lo, int32_t n,
                                     int32_t rows_per_member, float* d_y, int64_t y_stride,
                                     int64_t y_plane, int32_t math, void* d_work,
                                     size_t work_bytes, void* stream) {
    LinParams P;
    DeviceState* st = nullptr;
    int rc = make_params(&P, d_x, x_fmt, x_stride, x_plane, n_time, d_W, a, b, key, rank, sigma,
                         epoch, noise_reuse, tid_lo, n, rows_per_member, math, &st);
    if (rc || n == 0) return rc;
    return run_linear(P, st, d_y, y_stride, y_plane, d_work, work_bytes, stream,
                      "hses_perturbed_linear");
}

extern "C" size_t hses_perturbed_linear_t_workspace(int32_t a, int32_t b, int32_t rank, int32_t n,
                                                    int32_t rows_per_member, int32_t n_time,
                                                    int32_t math) {
    return hses_perturbed_linear_workspace(b, a, rank, n, rows_per_member, n_time, math);
}

extern "C" int hses_perturbed_linear_t(const void* d_x, int32_t x_fmt, int64_t x_stride,
                                       int64_t x_plane, int32_t n_time, const float* d_W,
                                       int32_t a, int32_t b, uint64_t key, int32_t rank,
                                       float sigma, int32_t epoch, int32_t noise_reuse,
                                       int32_t tid_lo, int32_t n, int32_t rows_per_member,
                                       float* d_y, int64_t y_stride, int64_t y_plane, int32_t math,
                                       void* d_work, size_t work_bytes, void* stream) {
    // The kernels' input width is the parameter's a, their output width its b.
    LinParams P;
    DeviceState* st = nullptr;
    int rc = make_params(&P, d_x, x_fmt, x_stride, x_plane, n_time, d_W, b, a, key, rank, sigma,
                         epoch, noise_reuse, tid_lo, n, rows_per_member, math, &st);
    if (rc || n == 0) return rc;
    P.tmm = 1;
    return run_linear(P, st, d_y, y_stride, y_plane, d_work, work_bytes, stream,
                      "hses_perturbed_linear_t");
}

// ---- factor record --------------------------------------------------------------
// The pair kernels can keep every pair's raw normals (B rows [0, b), A rows
// [b, a + b) of the stream, before any scale) for the ES update of the same
// parameter, which then reads them instead of drawing them again.

static int64_t record_pairs(int32_t tid_lo, int32_t n) {
    return n <= 0 ? 0 : (int64_t)(tid_lo + n - 1) / 2 - tid_lo / 2 + 1;
}

extern "C" size_t hses_factor_record_bytes(int32_t a, int32_t b, int32_t rank, int32_t tid_lo,
                                           int32_t n) {
    if (a < 1 || b < 1 || rank < 1 || tid_lo < 0 || n < 1) return 0;
    return (size_t)record_pairs(tid_lo, n) * (size_t)(a + b) * rank * sizeof(float);
}

static int check_record(const LinParams& P, const float* d_rec, size_t rec_bytes, const char* name) {
    HSES_REQUIRE(d_rec, "factor record is NULL");
    HSES_REQUIRE(P.r >= 32 && P.r % 16 == 0 && P.r <= 128,
                 std::string(name) + ": the factor record needs rank a multiple of 16 in "
                                     "[32, 128] and sigma != 0");
    HSES_REQUIRE(rec_bytes >= hses_factor_record_bytes(P.a, P.b, P.r, P.tid_lo, P.n),
                 std::string(name) + ": factor record smaller than hses_factor_record_bytes");
    return HSES_OK;
}

extern "C" int hses_perturbed_linear_rec(const void* d_x, int32_t x_fmt, int64_t x_stride,
                                         int64_t x_plane, int32_t n_time, const float* d_W,
                                         int32_t a, int32_t b, uint64_t key, int32_t rank,
                                         float sigma, int32_t epoch, int32_t noise_reuse,
                                         int32_t tid_lo, int32_t n, int32_t rows_per_member,
                                         float* d_y, int64_t y_stride, int64_t y_plane,
                                         int32_t math, void* d_work, size_t work_bytes,
                                         float* d_rec, size_t rec_bytes, void* stream) {
    LinParams P;
    DeviceState* st = nullptr;
    int rc = make_params(&P, d_x, x_fmt, x_stride, x_plane, n_time, d_W, a, b, key, rank, sigma,
                         epoch, noise_reuse, tid_lo, n, rows_per_member, math, &st);
    if (rc || n == 0) return rc;
    rc = check_record(P, d_rec, rec_bytes, "hses_perturbed_linear_rec");
    if (rc) return rc;
    HSES_REQUIRE(d_y, "NULL pointer");
    HSES_REQUIRE(rows_layout_ok(a, (int64_t)n * rows_per_member, n_time, y_stride, y_plane),
                 "y rows overlap (y_stride smaller than a row, or time planes overlap)");
    P.y = d_y;
    P.y_stride = y_stride;
    P.y_plane = y_plane;
    P.rec = d_rec;
    rc = launch_linear_pair(P, st, (hipStream_t)stream, d_work, work_bytes);
    if (rc == HSES_ERR_UNSUPPORTED)
        return set_error(HSES_ERR_UNSUPPORTED,
                         "hses_perturbed_linear_rec: the factor record needs the pair kernels "
                         "(bf16 math, a <= 128)");
    return rc;
}

static int linear_lif_impl(const void* d_x, int32_t x_fmt, int64_t x_stride, int64_t x_plane,
                           int32_t n_time, const float* d_W, int32_t a, int32_t b, uint64_t key,
                           int32_t rank, float sigma, int32_t epoch, int32_t noise_reuse,
                           int32_t tid_lo, int32_t n, int32_t rows_per_member, float tau_m,
                           float v_th, uint64_t* d_spikes, int64_t spk_stride, int64_t spk_plane,
                           float* d_rate, int64_t rate_stride, void* d_work, size_t work_bytes,
                           float* d_rec, size_t rec_bytes, void* stream,
                           const uint16_t* d_img = nullptr, size_t img_bytes = 0,
                           bool split = false, uint64_t* d_counts = nullptr,
                           int64_t counts_stride = 0) {
    HSES_REQUIRE(tau_m != 0.0f, "tau_m must be non-zero");
    LinParams P;
    DeviceState* st = nullptr;
    int rc = make_params(&P, d_x, x_fmt, x_stride, x_plane, n_time, d_W, a, b, key, rank, sigma,
                         epoch, noise_reuse, tid_lo, n, rows_per_member, HSES_MATH_BF16, &st);
    if (rc || n == 0) return rc;
    if (d_rec || rec_bytes) {
        rc = check_record(P, d_rec, rec_bytes, "hses_perturbed_linear_lif_rec");
        if (rc) return rc;
        P.rec = d_rec;
    }
    if (d_img && !split) {
        HSES_REQUIRE(img_bytes >= pair_image_bytes(a, b, P.r, tid_lo, n),
                     "hses_perturbed_linear_lif_pre: operand image smaller than "
                     "hses_pair_image_bytes");
    }
    if (split) P.math = HSES_MATH_F32X;
    HSES_REQUIRE(d_spikes || d_rate || d_counts, "spikes and rate are both NULL");
    const int64_t M = (int64_t)n * rows_per_member;
    HSES_REQUIRE(!d_spikes || rows_layout_ok((a + 63) / 64, M, n_time, spk_stride, spk_plane),
                 "spike rows overlap (spk_stride smaller than a row, or time planes overlap)");
    HSES_REQUIRE(!d_rate || rate_stride >= a, "rate_stride smaller than a row");
    HSES_REQUIRE(P.r > 0, "the fused kernel needs rank > 0 and sigma != 0");
    HSES_REQUIRE(n_time <= 64 && (n_time & (n_time - 1)) == 0, "n_time must be a power of two <= 64");
    HSES_REQUIRE(x_fmt == HSES_FMT_BITS, "the fused kernel takes bit-packed spikes (x_fmt BITS)");
    LifOut lif{d_spikes, spk_stride, spk_plane, d_rate, rate_stride,
               1.0f / tau_m /* snn.rs:59: dt / tau_m with dt = 1 */, v_th, d_counts, counts_stride};
    rc = launch_linear_pair(P, st, (hipStream_t)stream, d_work, work_bytes, &lif, d_img);
    if (rc == HSES_ERR_UNSUPPORTED)
        return set_error(HSES_ERR_UNSUPPORTED,
                         split ? "hses_perturbed_linear_lif_pre_x: needs rank a multiple of 16 <= 128, "
                                 "a <= 128, n_time <= 16 and b <= 896"
                         : d_img ? "hses_perturbed_linear_lif_pre: needs rank a multiple of 16 <= 128, "
                                   "a <= 128, n_time <= 16 and b <= 1024"
                                 : "hses_perturbed_linear_lif: needs rank a multiple of 16 <= 128 and a <= 128");
    return rc;
}

extern "C" int hses_perturbed_linear_lif(const void* d_x, int32_t x_fmt, int64_t x_stride,
                                         int64_t x_plane, int32_t n_time, const float* d_W,
                                         int32_t a, int32_t b, uint64_t key, int32_t rank,
                                         float sigma, int32_t epoch, int32_t noise_reuse,
                                         int32_t tid_lo, int32_t n, int32_t rows_per_member,
                                         float tau_m, float v_th, uint64_t* d_spikes,
                                         int64_t spk_stride, int64_t spk_plane, float* d_rate,
                                         int64_t rate_stride, void* d_work, size_t work_bytes,
                                         void* stream) {
    return linear_lif_impl(d_x, x_fmt, x_stride, x_plane, n_time, d_W, a, b, key, rank, sigma,
                           epoch, noise_reuse, tid_lo, n, rows_per_member, tau_m, v_th, d_spikes,
                           spk_stride, spk_plane, d_rate, rate_stride, d_work, work_bytes, nullptr,
                           0, stream);
}

extern "C" int hses_perturbed_linear_lif_rec(const void* d_x, int32_t x_fmt, int64_t x_stride,
                                             int64_t x_plane, int32_t n_time, const float* d_W,
                                             int32_t a, int32_t b, uint64_t key, int32_t rank,
                                             float sigma, int32_t epoch, int32_t noise_reuse,
                                             int32_t tid_lo, int32_t n, int32_t rows_per_member,
                                             float tau_m, float v_th, uint64_t* d_spikes,
                                             int64_t spk_stride, int64_t spk_plane, float* d_rate,
                                             int64_t rate_stride, void* d_work, size_t work_bytes,
                                             float* d_rec, size_t rec_bytes, void* stream) {
    HSES_REQUIRE(d_rec, "factor record is NULL");
    return linear_lif_impl(d_x, x_fmt, x_stride, x_plane, n_time, d_W, a, b, key, rank, sigma,
                           epoch, noise_reuse, tid_lo, n, rows_per_member, tau_m, v_th, d_spikes,
                           spk_stride, spk_plane, d_rate, rate_stride, d_work, work_bytes, d_rec,
                           rec_bytes, stream);
}

// ---- factors drawn ahead -----------------------------------------------------
// hses_pair_factors draws every pair's factors of a do_mm pair-kernel forward
// into the factor record and the bf16 B operand image; the *_pre forwards
// then read them instead of drawing, with the same operands, products and
// order as the *_rec forwards (so the same outputs, bit for bit).  The draw
// is a separate full-occupancy launch that a caller may put on another
// stream or issue ahead of the forward.

// The record and operand image of factors drawn ahead, checked from the
// arguments alone (before the device is touched).
static int check_drawn(int32_t a, int32_t b, int32_t rank, float sigma, int32_t tid_lo, int32_t n,
                       const float* d_rec, size_t rec_bytes, const void* d_img, size_t img_bytes,
                       const char* name, bool split = false, bool img_optional = false) {
    const int32_t r = (sigma != 0.0f) ? rank : 0;
    HSES_REQUIRE(a >= 1 && a <= 128,
                 std::string(name) + ": output width a must be in [1, 128] (the pair kernels)");
    HSES_REQUIRE(r >= 32 && r % 16 == 0 && r <= 128,
                 std::string(name) + ": factors drawn ahead need rank a multiple of 16 in "
                                     "[32, 128] and sigma != 0");
    HSES_REQUIRE(d_rec, std::string(name) + ": factor record is NULL");
    HSES_REQUIRE(rec_bytes >= hses_factor_record_bytes(a, b, r, tid_lo, n),
                 std::string(name) + ": factor record smaller than hses_factor_record_bytes");
    if (img_optional && !d_img && img_bytes == 0) return HSES_OK;  // the record alone
    HSES_REQUIRE(d_img, std::string(name) + ": operand image is NULL");
    if (split)
        HSES_REQUIRE(img_bytes >= pair_image_x_bytes(a, b, r, tid_lo, n),
                     std::string(name) + ": operand image smaller than hses_pair_image_x_bytes");
    else
        HSES_REQUIRE(img_bytes >= pair_image_bytes(a, b, r, tid_lo, n),
                     std::string(name) + ": operand image smaller than hses_pair_image_bytes");
    return HSES_OK;
}

extern "C" size_t hses_pair_image_bytes(int32_t a, int32_t b, int32_t rank, int32_t tid_lo,
                                        int32_t n) {
    if (a < 1 || b < 1 || rank < 1 || tid_lo < 0 || n < 1) return 0;
    return pair_image_bytes(a, b, rank, tid_lo, n);
}

static int pair_factors_impl(uint64_t key, int32_t rank, float sigma, int32_t epoch,
                             int32_t noise_reuse, int32_t tid_lo, int32_t n, int32_t a, int32_t b,
                             float* d_rec, size_t rec_bytes, uint16_t* d_img, size_t img_bytes,
                             void* stream, bool split) {
    HSES_REQUIRE(a >= 1 && b >= 1 && n >= 0 && rank >= 0, "bad sizes");
    HSES_REQUIRE(noise_reuse >= 0, "noise_reuse must be >= 0");
    HSES_REQUIRE(tid_lo >= 0 && (int64_t)tid_lo + n - 1 <= INT32_MAX, "thread id range");
    if (n == 0) return HSES_OK;
    int rc = check_drawn(a, b, rank, sigma, tid_lo, n, d_rec, rec_bytes, d_img, img_bytes,
                         split ? "hses_pair_factors_x" : "hses_pair_factors", split, true);
    if (rc) return rc;
    DeviceState* st;
    rc = get_state(&st);
    if (rc) return rc;
    LinParams P{};
    P.a = a;
    P.b = b;
    P.key = key;
    P.r = rank;
    P.bs = sigma / sqrtf((float)rank);  // eggroll.rs:433
    P.epoch = epoch;
    P.nreuse = noise_reuse;
    P.tid_lo = tid_lo;
    P.n = n;
    P.math = HSES_MATH_BF16;
    P.tables = st->d_tables;
    P.log_exc = st->d_log_exc;
    P.cos_exc = st->d_cos_exc;
    P.rec = d_rec;
    return launch_pair_gen(P, st, (hipStream_t)stream, d_img, split);
}

extern "C" int hses_pair_factors(uint64_t key, int32_t rank, float sigma, int32_t epoch,
                                 int32_t noise_reuse, int32_t tid_lo, int32_t n, int32_t a,
                                 int32_t b, float* d_rec, size_t rec_bytes, uint16_t* d_img,
                                 size_t img_bytes, void* stream) {
    return pair_factors_impl(key, rank, sigma, epoch, noise_reuse, tid_lo, n, a, b, d_rec,
                             rec_bytes, d_img, img_bytes, stream, false);
}

static int linear_pre_impl(const void* d_x, int32_t x_fmt, int64_t x_stride, int64_t x_plane,
                           int32_t n_time, const float* d_W, int32_t a, int32_t b, int32_t rank,
                           float sigma, int32_t tid_lo, int32_t n, int32_t rows_per_member,
                           float* d_y, int64_t y_stride, int64_t y_plane, void* d_work,
                           size_t work_bytes, const float* d_rec, size_t rec_bytes,
                           const uint16_t* d_img, size_t img_bytes, void* stream, bool split) {
    const char* name = split ? "hses_perturbed_linear_pre_x" : "hses_perturbed_linear_pre";
    if (n > 0 && tid_lo >= 0) {
        const int rc0 = check_drawn(a, b, rank, sigma, tid_lo, n, d_rec, rec_bytes, d_img,
                                    img_bytes, name, split);
        if (rc0) return rc0;
    }
    LinParams P;
    DeviceState* st = nullptr;
    int rc = make_params(&P, d_x, x_fmt, x_stride, x_plane, n_time, d_W, a, b, 0, rank, sigma, 0,
                         0, tid_lo, n, rows_per_member, HSES_MATH_BF16, &st);
    if (rc || n == 0) return rc;
    HSES_REQUIRE(d_y, "NULL pointer");
    HSES_REQUIRE(rows_layout_ok(a, (int64_t)n * rows_per_member, n_time, y_stride, y_plane),
                 "y rows overlap (y_stride smaller than a row, or time planes overlap)");
    P.y = d_y;
    P.y_stride = y_stride;
    P.y_plane = y_plane;
    P.rec = const_cast<float*>(d_rec);
    if (split) P.math = HSES_MATH_F32X;
    rc = launch_linear_pair(P, st, (hipStream_t)stream, d_work, work_bytes, nullptr, d_img);
    if (rc == HSES_ERR_UNSUPPORTED)
        return set_error(HSES_ERR_UNSUPPORTED,
                         split ? "hses_perturbed_linear_pre_x: needs bit-packed x (x_fmt BITS), "
                                 "a <= 128, rank a multiple of 16 in [32, 128] and b <= 896"
                               : "hses_perturbed_linear_pre: needs the pair kernels (a <= 128, rank a "
                                 "multiple of 16 in [32, 128])");
    return rc;
}

extern "C" int hses_perturbed_linear_pre(const void* d_x, int32_t x_fmt, int64_t x_stride,
                                         int64_t x_plane, int32_t n_time, const float* d_W,
                                         int32_t a, int32_t b, int32_t rank, float sigma,
                                         int32_t tid_lo, int32_t n, int32_t rows_per_member,
                                         float* d_y, int64_t y_stride, int64_t y_plane,
                                         void* d_work, size_t work_bytes, const float* d_rec,
                                         size_t rec_bytes, const uint16_t* d_img,
                                         size_t img_bytes, void* stream) {
    return linear_pre_impl(d_x, x_fmt, x_stride, x_plane, n_time, d_W, a, b, rank, sigma, tid_lo,
                           n, rows_per_member, d_y, y_stride, y_plane, d_work, work_bytes, d_rec,
                           rec_bytes, d_img, img_bytes, stream, false);
}

extern "C" int hses_perturbed_linear_lif_pre(const void* d_x, int32_t x_fmt, int64_t x_stride,
                                             int64_t x_plane, int32_t n_time, const float* d_W,
                                             int32_t a, int32_t b, int32_t rank, float sigma,
                                             int32_t tid_lo, int32_t n, int32_t rows_per_member,
                                             float tau_m, float v_th, uint64_t* d_spikes,
                                             int64_t spk_stride, int64_t spk_plane, float* d_rate,
                                             int64_t rate_stride, void* d_work, size_t work_bytes,
                                             const float* d_rec, size_t rec_bytes,
                                             const uint16_t* d_img, size_t img_bytes,
                                             void* stream) {
    if (n > 0 && tid_lo >= 0) {
        const int rc = check_drawn(a, b, rank, sigma, tid_lo, n, d_rec, rec_bytes, d_img,
                                   img_bytes, "hses_perturbed_linear_lif_pre");
        if (rc) return rc;
    }
    return linear_lif_impl(d_x, x_fmt, x_stride, x_plane, n_time, d_W, a, b, 0, rank, sigma, 0, 0,
                           tid_lo, n, rows_per_member, tau_m, v_th, d_spikes, spk_stride,
                           spk_plane, d_rate, rate_stride, d_work, work_bytes,
                           const_cast<float*>(d_rec), rec_bytes, stream, d_img, img_bytes);
}

// ---- the split (fp32-accurate) forwards -------------------------------------
// The *_pre forwards on a split operand image (hses_pair_image_x) and W split
// the same way, as fp16 MFMA products of high and low parts.

extern "C" size_t hses_pair_image_x_bytes(int32_t a, int32_t b, int32_t rank, int32_t tid_lo,
                                          int32_t n) {
    if (a < 1 || b < 1 || rank < 1 || tid_lo < 0 || n < 1) return 0;
    return pair_image_x_bytes(a, b, rank, tid_lo, n);
}

extern "C" int hses_pair_image_x(int32_t a, int32_t b, int32_t rank, float sigma, int32_t tid_lo,
                                 int32_t n, const float* d_rec, size_t rec_bytes, uint16_t* d_img,
                                 size_t img_bytes, void* stream) {
    HSES_REQUIRE(a >= 1 && b >= 1 && n >= 0 && rank >= 0, "bad sizes");
    HSES_REQUIRE(tid_lo >= 0 && (int64_t)tid_lo + n - 1 <= INT32_MAX, "thread id range");
    if (n == 0) return HSES_OK;
    int rc = check_drawn(a, b, rank, sigma, tid_lo, n, d_rec, rec_bytes, d_img, img_bytes,
                         "hses_pair_image_x", true);
    if (rc) return rc;
    DeviceState* st;
    rc = get_state(&st);
    if (rc) return rc;
    return launch_pair_image_x(d_rec, a, b, rank, sigma / sqrtf((float)rank) /* eggroll.rs:433 */,
                               tid_lo, n, d_img, (hipStream_t)stream);
}

extern "C" int hses_pair_factors_x(uint64_t key, int32_t rank, float sigma, int32_t epoch,
                                   int32_t noise_reuse, int32_t tid_lo, int32_t n, int32_t a,
                                   int32_t b, float* d_rec, size_t rec_bytes, uint16_t* d_img,
                                   size_t img_bytes, void* stream) {
    return pair_factors_impl(key, rank, sigma, epoch, noise_reuse, tid_lo, n, a, b, d_rec,
                             rec_bytes, d_img, img_bytes, stream, true);
}

extern "C" int hses_perturbed_linear_pre_x(const void* d_x, int32_t x_fmt, int64_t x_stride,
                                           int64_t x_plane, int32_t n_time, const float* d_W,
                                           int32_t a, int32_t b, int32_t rank, float sigma,
                                           int32_t tid_lo, int32_t n, int32_t rows_per_member,
                                           float* d_y, int64_t y_stride, int64_t y_plane,
                                           void* d_work, size_t work_bytes, const float* d_rec,
                                           size_t rec_bytes, const uint16_t* d_img,
                                           size_t img_bytes, void* stream) {
    return linear_pre_impl(d_x, x_fmt, x_stride, x_plane, n_time, d_W, a, b, rank, sigma, tid_lo,
                           n, rows_per_member, d_y, y_stride, y_plane, d_work, work_bytes, d_rec,
                           rec_bytes, d_img, img_bytes, stream, true);
}

// ---- member weights ------------------------------------------------------------
// W_m = W + sign_m (sigma / sqrt(r)) A_m B_m^T of every member from the factor
// record (hses_member_weights), then the forwards y = x W_m^T on them
// (hses_perturbed_linear_mw, hses_perturbed_linear_lif_mw).

static int check_mw_math(int32_t math, const char* name) {
    HSES_REQUIRE(math == HSES_MATH_BF16 || math == HSES_MATH_F32X,
                 std::string(name) + ": math must be HSES_MATH_BF16 or HSES_MATH_F32X");
    return HSES_OK;
}

extern "C" size_t hses_member_weights_bytes(int32_t a, int32_t b, int32_t n, int32_t math) {
    if (math != HSES_MATH_BF16 && math != HSES_MATH_F32X) return 0;
    return member_weights_bytes(a, b, n, math == HSES_MATH_F32X);
}

extern "C" int hses_member_weights(const float* d_W, int32_t a, int32_t b, int32_t rank,
                                   float sigma, int32_t tid_lo, int32_t n, const float* d_rec,
                                   size_t rec_bytes, int32_t math, uint16_t* d_wm,
                                   size_t wm_bytes, void* stream) {
    HSES_REQUIRE(a >= 1 && b >= 1 && n >= 0 && rank >= 0, "bad sizes");
    HSES_REQUIRE(tid_lo >= 0 && (int64_t)tid_lo + n - 1 <= INT32_MAX, "thread id range");
    int rc = check_mw_math(math, "hses_member_weights");
    if (rc || n == 0) return rc;
    rc = check_drawn(a, b, rank, sigma, tid_lo, n, d_rec, rec_bytes, nullptr, 0,
                     "hses_member_weights", false, true);
    if (rc) return rc;
    HSES_REQUIRE(d_W && d_wm, "NULL pointer");
    HSES_REQUIRE(wm_bytes >= member_weights_bytes(a, b, n, math == HSES_MATH_F32X),
                 "hses_member_weights: buffer smaller than hses_member_weights_bytes");
    DeviceState* st;
    rc = get_state(&st);
    if (rc) return rc;
    return launch_member_weights(d_W, d_rec, a, b, rank, sigma / sqrtf((float)rank) /* eggroll.rs:433 */,
                                 tid_lo, n, math == HSES_MATH_F32X, d_wm, (hipStream_t)stream);
}

// Checks shared by the two member-weight forwards; fills P (x, sizes, the
// weights).
static int mw_params(LinParams* P, DeviceState** st, const void* d_x, int32_t x_fmt,
                     int64_t x_stride, int64_t x_plane, int32_t n_time, int32_t a, int32_t b,
                     int32_t tid_lo, int32_t n, int32_t rows_per_member, int32_t math,
                     const uint16_t* d_wm, size_t wm_bytes, const char* name) {
    int rc = check_mw_math(math, name);
    if (rc) return rc;
    HSES_REQUIRE(x_fmt == HSES_FMT_BITS, std::string(name) + ": x must be bit-packed (x_fmt BITS)");
    HSES_REQUIRE(a >= 1 && a <= 128 && b >= 1 && b <= 1024,
                 std::string(name) + ": needs a <= 128 and b <= 1024");
    HSES_REQUIRE(math == HSES_MATH_F32X || b > 64,
                 std::string(name) + ": bf16 member weights need b > 64");
    // a stand-in W pointer: make_params checks it, the kernels read d_wm
    rc = make_params(P, d_x, x_fmt, x_stride, x_plane, n_time, reinterpret_cast<const float*>(d_wm),
                     a, b, 0, 0, 0.0f, 0, 0, tid_lo, n, rows_per_member, HSES_MATH_BF16, st);
    if (rc || n == 0) return rc;
    HSES_REQUIRE(((int64_t)n_time * rows_per_member) % 256 == 0,
                 std::string(name) + ": rows per member (n_time x rows_per_member) must be a "
                                     "multiple of 256");
    HSES_REQUIRE(wm_bytes >= member_weights_bytes(a, b, n, math == HSES_MATH_F32X),
                 std::string(name) + ": weights smaller than hses_member_weights_bytes");
    P->math = math;
    P->wm = d_wm;
    P->wm_stride = (int64_t)(member_weights_bytes(a, b, 1, math == HSES_MATH_F32X) / 2);
    return HSES_OK;
}

extern "C" int hses_perturbed_linear_mw(const void* d_x, int32_t x_fmt, int64_t x_stride,
                                        int64_t x_plane, int32_t n_time, int32_t a, int32_t b,
                                        int32_t tid_lo, int32_t n, int32_t rows_per_member,
                                        int32_t math, const uint16_t* d_wm, size_t wm_bytes,
                                        float* d_y, int64_t y_stride, int64_t y_plane,
                                        void* stream) {
    LinParams P;
    DeviceState* st = nullptr;
    int rc = mw_params(&P, &st, d_x, x_fmt, x_stride, x_plane, n_time, a, b, tid_lo, n,
                       rows_per_member, math, d_wm, wm_bytes, "hses_perturbed_linear_mw");
    if (rc || n == 0) return rc;
    HSES_REQUIRE(d_y, "NULL pointer");
    HSES_REQUIRE(rows_layout_ok(a, (int64_t)n * rows_per_member, n_time, y_stride, y_plane),
                 "y rows overlap (y_stride smaller than a row, or time planes overlap)");
    P.y = d_y;
    P.y_stride = y_stride;
    P.y_plane = y_plane;
    rc = launch_linear_mw(P, st, (hipStream_t)stream, nullptr);
    if (rc == HSES_ERR_UNSUPPORTED)
        return set_error(HSES_ERR_UNSUPPORTED, "hses_perturbed_linear_mw: unsupported shape");
    return rc;
}

extern "C" int hses_perturbed_linear_lif_mw(
    const void* d_x, int32_t x_fmt, int64_t x_stride, int64_t x_plane, int32_t n_time, int32_t a,
    int32_t b, int32_t tid_lo, int32_t n, int32_t rows_per_member, float tau_m, float v_th,
    int32_t math, const uint16_t* d_wm, size_t wm_bytes, uint64_t* d_spikes, int64_t spk_stride,
    int64_t spk_plane, float* d_rate, int64_t rate_stride, uint64_t* d_counts,
    int64_t counts_stride, void* stream) {
    HSES_REQUIRE(tau_m != 0.0f, "tau_m must be non-zero");
    HSES_REQUIRE(n_time >= 1 && n_time <= 16 && (n_time & (n_time - 1)) == 0,
                 "hses_perturbed_linear_lif_mw: n_time must be a power of two <= 16");
    LinParams P;
    DeviceState* st = nullptr;
    int rc = mw_params(&P, &st, d_x, x_fmt, x_stride, x_plane, n_time, a, b, tid_lo, n,
                       rows_per_member, math, d_wm, wm_bytes, "hses_perturbed_linear_lif_mw");
    if (rc || n == 0) return rc;
    HSES_REQUIRE(d_spikes || d_rate || d_counts, "spikes, rate and counts are all NULL");
    HSES_REQUIRE(!(d_rate && d_counts), "rate and counts are exclusive");
    const int64_t M = (int64_t)n * rows_per_member;
    HSES_REQUIRE(!d_spikes || rows_layout_ok((a + 63) / 64, M, n_time, spk_stride, spk_plane),
                 "spike rows overlap (spk_stride smaller than a row, or time planes overlap)");
    HSES_REQUIRE(!d_rate || rate_stride >= a, "rate_stride smaller than a row");
    int32_t planes = 1;
    while ((1 << (planes - 1)) < n_time) ++planes;
    HSES_REQUIRE(!d_counts || counts_stride >= (int64_t)planes * ((a + 63) / 64),
                 "counts_stride smaller than a row's count planes");
    LifOut lif{d_spikes, spk_stride, spk_plane, d_rate, rate_stride,
               1.0f / tau_m /* snn.rs:59: dt / tau_m with dt = 1 */, v_th, d_counts, counts_stride};
    rc = launch_linear_mw(P, st, (hipStream_t)stream, &lif);
    if (rc == HSES_ERR_UNSUPPORTED)
        return set_error(HSES_ERR_UNSUPPORTED, "hses_perturbed_linear_lif_mw: unsupported shape");
    return rc;
}

extern "C" int hses_perturbed_readout_counts(const uint64_t* d_counts, int64_t counts_stride,
                                             int32_t n_time, const float* d_W, int32_t a,
                                             int32_t b, int32_t rank, float sigma, int32_t tid_lo,
                                             int32_t n, int32_t rows_per_member,
                                             const float* d_rec, size_t rec_bytes, float* d_y,
                                             int64_t y_stride, void* stream) {
    HSES_REQUIRE(a >= 1 && b >= 1 && n >= 0 && rank >= 1 && rows_per_member >= 1, "bad sizes");
    HSES_REQUIRE(tid_lo >= 0 && (int64_t)tid_lo + n - 1 <= INT32_MAX, "thread id range");
    HSES_REQUIRE(n_time >= 1 && n_time <= 16 && (n_time & (n_time - 1)) == 0,
                 "hses_perturbed_readout_counts: n_time must be a power of two <= 16");
    HSES_REQUIRE(a <= 32 && b <= 128 && rows_per_member <= 128,
                 "hses_perturbed_readout_counts: a <= 32, b <= 128 and rows_per_member <= 128");
    HSES_REQUIRE(readout_counts_lds(a, b, rank) <= 160 * 1024,
                 "hses_perturbed_readout_counts: rank * (a + b) too large for LDS");
    if (n == 0) return HSES_OK;
    int rc = check_drawn(a, b, rank, sigma, tid_lo, n, d_rec, rec_bytes, nullptr, 0,
                         "hses_perturbed_readout_counts", false, true);
    if (rc) return rc;
    HSES_REQUIRE(d_counts && d_W && d_y, "NULL pointer");
    int32_t planes = 1;
    while ((1 << (planes - 1)) < n_time) ++planes;
    HSES_REQUIRE(counts_stride >= (int64_t)planes * ((b + 63) / 64),
                 "counts_stride smaller than a row's count planes");
    HSES_REQUIRE(y_stride >= a, "y_stride smaller than a row");
    DeviceState* st;
    rc = get_state(&st);
    if (rc) return rc;
    rc = launch_readout_counts(d_counts, counts_stride, n_time, d_W, a, b, rank,
                               sigma / sqrtf((float)rank) /* eggroll.rs:433 */, tid_lo, n,
                               rows_per_member, d_rec, d_y, y_stride, (hipStream_t)stream);
    if (rc == HSES_ERR_UNSUPPORTED)
        return set_error(HSES_ERR_UNSUPPORTED, "hses_perturbed_readout_counts: unsupported shape");
    return rc;
}

extern "C" int hses_perturbed_linear_lif_counts_pre_x(
    const void* d_x, int32_t x_fmt, int64_t x_stride, int64_t x_plane, int32_t n_time,
    const float* d_W, int32_t a, int32_t b, int32_t rank, float sigma, int32_t tid_lo, int32_t n,
    int32_t rows_per_member, float tau_m, float v_th, uint64_t* d_counts, int64_t counts_stride,
    void* d_work, size_t work_bytes, const float* d_rec, size_t rec_bytes, const uint16_t* d_img,
    size_t img_bytes, void* stream) {
    if (n > 0 && tid_lo >= 0) {
        const int rc = check_drawn(a, b, rank, sigma, tid_lo, n, d_rec, rec_bytes, d_img,
                                   img_bytes, "hses_perturbed_linear_lif_counts_pre_x", true);
        if (rc) return rc;
    }
    HSES_REQUIRE(d_counts, "count planes are NULL");
    HSES_REQUIRE(n_time >= 1 && n_time <= 16 && (n_time & (n_time - 1)) == 0,
                 "hses_perturbed_linear_lif_counts_pre_x: n_time must be a power of two <= 16");
    int32_t planes = 1;
    while ((1 << (planes - 1)) < n_time) ++planes;
    HSES_REQUIRE(counts_stride >= (int64_t)planes * ((a + 63) / 64),
                 "counts_stride smaller than a row's count planes");
    return linear_lif_impl(d_x, x_fmt, x_stride, x_plane, n_time, d_W, a, b, 0, rank, sigma, 0, 0,
                           tid_lo, n, rows_per_member, tau_m, v_th, nullptr, 0, 0, nullptr, 0,
                           d_work, work_bytes, const_cast<float*>(d_rec), rec_bytes, stream, d_img,
                           img_bytes, true, d_counts, counts_stride);
}

extern "C" int hses_perturbed_linear_lif_pre_x(
    const void* d_x, int32_t x_fmt, int64_t x_stride, int64_t x_plane, int32_t n_time,
    const float* d_W, int32_t a, int32_t b, int32_t rank, float sigma, int32_t tid_lo, int32_t n,
    int32_t rows_per_member, float tau_m, float v_th, uint64_t* d_spikes, int64_t spk_stride,
    int64_t spk_plane, float* d_rate, int64_t rate_stride, void* d_work, size_t work_bytes,
    const float* d_rec, size_t rec_bytes, const uint16_t* d_img, size_t img_bytes, void* stream) {
    if (n > 0 && tid_lo >= 0) {
        const int rc = check_drawn(a, b, rank, sigma, tid_lo, n, d_rec, rec_bytes, d_img,
                                   img_bytes, "hses_perturbed_linear_lif_pre_x", true);
        if (rc) return rc;
    }
    return linear_lif_impl(d_x, x_fmt, x_stride, x_plane, n_time, d_W, a, b, 0, rank, sigma, 0, 0,
                           tid_lo, n, rows_per_member, tau_m, v_th, d_spikes, spk_stride,
                           spk_plane, d_rate, rate_stride, d_work, work_bytes,
                           const_cast<float*>(d_rec), rec_bytes, stream, d_img, img_bytes, true);
}

extern "C" int hses_perturbed_linear_act(const void* d_x, int32_t x_fmt, int64_t x_stride,
                                         int64_t x_plane, int32_t n_time, const float* d_W,
                                         int32_t a, int32_t b, uint64_t key, int32_t rank,
                                         float sigma, int32_t epoch, int32_t noise_reuse,
                                         int32_t tid_lo, int32_t n, int32_t rows_per_member,
                                         void* d_y, int64_t y_stride, int64_t y_plane,
                                         int32_t math, int32_t transposed, int32_t act,
                                         int32_t y_fmt, void* d_work, size_t work_bytes,
                                         void* stream) {
    HSES_REQUIRE(transposed == 0 || transposed == 1, "transposed must be 0 or 1");
    LinParams P;
    DeviceState* st = nullptr;
    // do_Tmm: the kernels' input width is the parameter's a, their output width its b
    int rc = transposed ? make_params(&P, d_x, x_fmt, x_stride, x_plane, n_time, d_W, b, a, key,
                                      rank, sigma, epoch, noise_reuse, tid_lo, n, rows_per_member,
                                      math, &st)
                        : make_params(&P, d_x, x_fmt, x_stride, x_plane, n_time, d_W, a, b, key,
                                      rank, sigma, epoch, noise_reuse, tid_lo, n, rows_per_member,
                                      math, &st);
    if (rc || n == 0) return rc;
    P.tmm = transposed;
    return run_linear(P, st, static_cast<float*>(d_y), y_stride, y_plane, d_work, work_bytes,
                      stream, "hses_perturbed_linear_act", act, y_fmt);
}
