// linear_f32.hip -- fp32 perturbed forward y = x W^T + (x B_m) A_m^T for small ranks.
//
// Reference: do_mm_impl (burn_impl/hyperscalees-noiser/src/eggroll.rs:419-446)
// and lora_linear_batched (burn_impl/hyperscalees-models/src/snn.rs:665-685).
//
// Two launches:
//   k_factors   every member's B_m (stream rows [0, b)) and scaled A_m (rows
//             [b, a + b)) into the workspace, each row drawn once.
//   k_gemm_f32  y = x W^T with fp32 MFMA (32x32x2) over 128-row x BN-column
//             tiles, K in chunks of 32 staged through double-buffered LDS with
//             the chunk's B_m rows beside them; each thread also accumulates
//             x B_m for its row on the vector ALU from the staged chunk, and the
//             epilogue adds (x B_m) A_m^T with the tile's A_m rows.
// The LDS copy of a chunk stores each row's 32 k values as the even k then the
// odd k, so a lane (row l % 32, k-group l / 32 of the 32x32x2 MFMA) reads its
// 16 k-steps of a chunk with four 16-byte loads.
#include <math.h>

#include "linear_common.h"
#include "noise_dev.h"
#include "runtime.h"

namespace hses {

constexpr int KF_BM = 128, KF_BK = 32, KF_THREADS = 256;
constexpr int KF_XP = 36;          // LDS pitch of a staged row (floats): 16 even k, 16 odd k, pad
constexpr int KF_AMAX = 8192;      // floats of A rows a workgroup keeps for its epilogue
constexpr int KF_RMAX = 16;        // ranks handled

typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16 mfma32x2(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Value k of row `off` of x in fp32 (k < b checked by the caller).
template <int XFMT>
__device__ __forceinline__ float x_at(const void* x, int64_t off, int32_t k) {
    if constexpr (XFMT == HSES_FMT_BITS) {
        const uint64_t w = static_cast<const uint64_t*>(x)[off + (k >> 6)];
        return (float)((w >> (k & 63)) & 1ull);
    } else if constexpr (XFMT == HSES_FMT_BF16) {
        return bf2f(static_cast<const uint16_t*>(x)[off + k]);
    } else {
        return static_cast<const float*>(x)[off + k];
    }
}

// ---- k_factors -------------------------------------------------------------------
// F[m] = the member's (a + b) x r stream rows as drawn, except that the
// rows carrying sign * sigma / sqrt(r) are scaled: do_mm's A rows [b, a + b),
// do_Tmm's input-side rows [a, a + b) (with a the output width).  A thread
// draws rows [q rc, q rc + rc) of one member after one jump to the group's start.
__global__ __launch_bounds__(256) void k_factors(LinParams P, int32_t rc, int32_t groups,
                                                 float* __restrict__ F) {
    __shared__ BmTables t;
    load_bm_tables(&t, P.tables);
    __syncthreads();
    const int64_t item = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (item >= (int64_t)P.n * groups) return;
    const int32_t m = (int32_t)(item / groups), q = (int32_t)(item % groups);
    const int32_t r = P.r, rows = P.a + P.b, row0 = q * rc;
    float sign;
    const uint64_t seed = member_seed(P.key, P.epoch, P.nreuse, P.tid_lo + m, &sign);
    const float sc = sign * P.bs;
    uint64_t s = row_start_state(seed, q, P.jump);
    const NoiseCtx ctx{&t, P.log_exc, P.cos_exc};
    float* dst = F + ((int64_t)m * rows + row0) * r;
    const int32_t split = ((P.tmm ? P.a : P.b) - row0) * r;  // normals before the first scaled row
    bm_run(s, min(rc, rows - row0) * r, ctx,
           [&](int32_t i, float v) { dst[i] = i >= split ? v * sc : v; });
}

// ---- k_gemm_f32 ------------------------------------------------------------------
// NT 32-column MFMA tiles per wave (BN = 32 NT); four waves of 32 rows.  RK is
// the rank padded to 1, 4, 8 or 16 (the LDS copies of B_m and A_m rows hold RK
// values per row, zero past r).
template <int XFMT, int NT, int RK>
__global__ __launch_bounds__(KF_THREADS) void k_gemm_f32(LinParams P, const float* __restrict__ F,
                                                         int32_t bch) {
    constexpr int BN = 32 * NT;
    extern __shared__ __align__(16) unsigned char smem[];
    // Two staging buffers, each: 128 x rows, BN W rows (KF_XP floats each), then
    // the chunk's B_m rows of the tile's members ([lm][32][RK]).  After them the
    // tile's A_m rows ([lm][BN][RK]).  bch (floats of a chunk's B_m rows, 0
    // without noise) is the host's, which sized the LDS.
    const int32_t bufsz = (KF_BM + BN) * KF_XP + bch;
    float* buf = reinterpret_cast<float*>(smem);
    // one staging buffer when K is a single chunk (b <= 32), else two
    float* As = buf + (P.b > KF_BK ? 2 : 1) * bufsz;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int32_t lc = lane & 31, kh = lane >> 5;
    // Tile of this workgroup: workgroups are dealt to the 8 XCDs in turn, so
    // XCD x gets the contiguous tile range x * nb / 8 .. with the column tiles
    // of a row tile adjacent: the workgroups that read the same x rows run on
    // one XCD together and share its L2.
    int64_t L0;
    int32_t o0;
    {
        const uint32_t nb = gridDim.x, g = blockIdx.x, xcd = g & 7u, j = g >> 3;
        const uint32_t q = nb >> 3, rem = nb & 7u;
        const uint32_t ncol = (uint32_t)((P.a + BN - 1) / BN);
        const uint32_t t = ncol == 1 ? g  // one column tile: no x rows are shared
                           : xcd < rem ? xcd * (q + 1) + j : rem * (q + 1) + (xcd - rem) * q + j;
        L0 = (int64_t)(t / ncol) * KF_BM;
        o0 = (int32_t)(t % ncol) * BN;
    }
    const int32_t ct = min(BN, P.a - o0);
    const int32_t r = P.r, b = P.b;
    const int32_t rows_here = (int32_t)min<int64_t>(KF_BM, P.total - L0);
    const TileRows tr(P, L0);
    const int32_t m_first = tr.m_first;
    const int32_t nm = tr.member(P, rows_here - 1) + 1;
    const bool noisy = r > 0;
    const int64_t fpitch = (int64_t)(P.a + b) * r;  // floats of one member's factors
    const float* Fm = F + (int64_t)m_first * fpitch;

    // ---- A rows of the tile's members: F rows b + o0 .. b + o0 + ct ------------
    if (noisy) {
        for (int32_t i = tid; i < nm * BN * RK; i += KF_THREADS) {
            const int32_t c = i % RK, o = (i / RK) % BN, lm = i / (RK * BN);
            As[i] = (c < r && o < ct) ? Fm[lm * fpitch + (int64_t)(b + o0 + o) * r + c] : 0.0f;
        }
    }

    // ---- staging: thread -> x row tid / 2 (16 k), W row tid * BN / 256 ----------
    const int xr = tid >> 1, xk = (tid & 1) * 16;
    const int64_t Lx = L0 + xr;
    const bool xvalid = Lx < P.total;
    const int64_t xoff = xvalid ? tr.offset(P, xr, P.x_stride, P.x_plane) : 0;
    const int32_t xlm = xvalid ? tr.member(P, xr) : 0;  // the x row's member in the tile
    constexpr int WPT = BN * KF_BK / KF_THREADS;  // W values per thread: 16, 8 or 4
    constexpr int WTPR = KF_BK / WPT;             // threads per W row
    const int wr = tid / WTPR, wk = (tid % WTPR) * WPT;
    const int32_t wo = o0 + wr;
    const bool wvalid = wo < P.a;
    const float* wrow = P.W + (size_t)(wvalid ? wo : 0) * b;
    constexpr int BPT = 8;  // B_m chunk values per thread (bch <= 8 * 256)
    float xv[16], wv[WPT], bv[BPT];
    auto load_chunk = [&](int32_t k0) {
        if constexpr (XFMT == HSES_FMT_BITS) {
            uint32_t bits = 0;
            const int32_t k = k0 + xk;
            if (xvalid && k < b) {
                const uint64_t w = static_cast<const uint64_t*>(P.x)[xoff + (k >> 6)];
                bits = (uint32_t)(w >> (k & 63)) & 0xffffu;
                if (b - k < 16) bits &= (1u << (b - k)) - 1u;
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) xv[i] = (float)((bits >> i) & 1u);
        } else {
            const int32_t k = k0 + xk;
            bool vec = xvalid && k + 16 <= b;
            if constexpr (XFMT == HSES_FMT_F32) {
                const float* xp = static_cast<const float*>(P.x) + xoff + k;
                if (vec && (reinterpret_cast<uintptr_t>(xp) & 15) == 0) {
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        *reinterpret_cast<float4*>(xv + 4 * q) = reinterpret_cast<const float4*>(xp)[q];
                } else {
                    vec = false;
                }
            } else {
                const uint16_t* xp = static_cast<const uint16_t*>(P.x) + xoff + k;
                if (vec && (reinterpret_cast<uintptr_t>(xp) & 15) == 0) {
#pragma unroll
                    for (int q = 0; q < 2; ++q) {
                        const uint4 u = reinterpret_cast<const uint4*>(xp)[q];
                        const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            xv[8 * q + 2 * e] = __uint_as_float(w4[e] << 16);
                            xv[8 * q + 2 * e + 1] = __uint_as_float(w4[e] & 0xffff0000u);
                        }
                    }
                } else {
                    vec = false;
                }
            }
            if (!vec) {
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    xv[i] = (xvalid && k + i < b) ? x_at<XFMT>(P.x, xoff, k + i) : 0.0f;
            }
        }
        {
            const int32_t k = k0 + wk;
            const float* wp = wrow + k;
            if (wvalid && k + WPT <= b && (reinterpret_cast<uintptr_t>(wp) & 15) == 0) {
#pragma unroll
                for (int q = 0; q < WPT / 4; ++q)
                    *reinterpret_cast<float4*>(wv + 4 * q) = reinterpret_cast<const float4*>(wp)[q];
            } else {
#pragma unroll
                for (int i = 0; i < WPT; ++i) wv[i] = (wvalid && k + i < b) ? wp[i] : 0.0f;
            }
        }
        if (noisy) {
#pragma unroll
            for (int j = 0; j < BPT; ++j) {
                const int32_t e = tid + KF_THREADS * j;  // [lm][kk][c] of the chunk
                const int32_t c = e % RK, kk = (e / RK) % KF_BK, lm = e / (RK * KF_BK);
                bv[j] = (e < bch && lm < nm && c < r && k0 + kk < b)
                            ? Fm[lm * fpitch + (int64_t)(k0 + kk) * r + c]
                            : 0.0f;
            }
        }
    };
    // even k to [0, 16), odd k to [16, 32) of the row, by k / 2
    auto store_chunk = [&](float* B) {
        float* xd = B + xr * KF_XP + (xk >> 1);
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
            xd[i >> 1] = xv[i];
            xd[16 + (i >> 1)] = xv[i + 1];
        }
        float* wd = B + (KF_BM + wr) * KF_XP + (wk >> 1);
#pragma unroll
        for (int i = 0; i < WPT; i += 2) {
            wd[i >> 1] = wv[i];
            wd[16 + (i >> 1)] = wv[i + 1];
        }
        if (noisy) {
            float* bd = B + (KF_BM + BN) * KF_XP;
#pragma unroll
            for (int j = 0; j < BPT; ++j) {
                const int32_t e = tid + KF_THREADS * j;
                if (e < bch) bd[e] = bv[j];
            }
        }
    };

    f32x16 acc[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[j][e] = 0.0f;
    float xb[RK];  // this thread's half of (x B_m) for row xr
#pragma unroll
    for (int c = 0; c < RK; ++c) xb[c] = 0.0f;

    const int32_t nch = (b + KF_BK - 1) / KF_BK;
    load_chunk(0);
    store_chunk(buf);
    __syncthreads();
    for (int32_t kc = 0; kc < nch; ++kc) {
        const float* B = buf + (kc & 1) * bufsz;
        if (kc + 1 < nch) load_chunk((kc + 1) * KF_BK);
        const float* ap = B + (wave * 32 + lc) * KF_XP + 16 * kh;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            float af[8], bfr[NT][8];
            *reinterpret_cast<float4*>(af) = *reinterpret_cast<const float4*>(ap + 8 * half);
            *reinterpret_cast<float4*>(af + 4) = *reinterpret_cast<const float4*>(ap + 8 * half + 4);
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                const float* bp = B + (KF_BM + 32 * j + lc) * KF_XP + 16 * kh + 8 * half;
                *reinterpret_cast<float4*>(bfr[j]) = *reinterpret_cast<const float4*>(bp);
                *reinterpret_cast<float4*>(bfr[j] + 4) = *reinterpret_cast<const float4*>(bp + 4);
            }
#pragma unroll
            for (int s = 0; s < 8; ++s)
#pragma unroll
                for (int j = 0; j < NT; ++j) acc[j] = mfma32x2(af[s], bfr[j][s], acc[j]);
        }
        if (noisy) {
            // x B_m over this thread's 16 k: even k xk + 2 i at [xk / 2 + i], odd at 16 + ..
            const float* xs = B + xr * KF_XP + (xk >> 1);
            const float* bs = B + (KF_BM + BN) * KF_XP + (xlm * KF_BK + xk) * RK;
            float ev[8], od[8];
            *reinterpret_cast<float4*>(ev) = *reinterpret_cast<const float4*>(xs);
            *reinterpret_cast<float4*>(ev + 4) = *reinterpret_cast<const float4*>(xs + 4);
            *reinterpret_cast<float4*>(od) = *reinterpret_cast<const float4*>(xs + 16);
            *reinterpret_cast<float4*>(od + 4) = *reinterpret_cast<const float4*>(xs + 20);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                float be[RK], bo[RK];
                if constexpr (RK == 1) {
                    be[0] = bs[2 * i];
                    bo[0] = bs[2 * i + 1];
                } else {
#pragma unroll
                    for (int q = 0; q < RK / 4; ++q) {
                        *reinterpret_cast<float4*>(be + 4 * q) =
                            *reinterpret_cast<const float4*>(bs + (2 * i) * RK + 4 * q);
                        *reinterpret_cast<float4*>(bo + 4 * q) =
                            *reinterpret_cast<const float4*>(bs + (2 * i + 1) * RK + 4 * q);
                    }
                }
#pragma unroll
                for (int c = 0; c < RK; ++c) {
                    xb[c] = __builtin_fmaf(ev[i], be[c], xb[c]);
                    xb[c] = __builtin_fmaf(od[i], bo[c], xb[c]);
                }
            }
        }
        if (kc + 1 < nch) store_chunk(buf + ((kc + 1) & 1) * bufsz);
        __syncthreads();
    }

    // ---- epilogue: y = x W^T + (x B_m) A_m^T -----------------------------------
    float* XBs = buf;  // [128][RK]; the staging buffers are free after the last barrier
    if (noisy) {
#pragma unroll
        for (int c = 0; c < RK; ++c) {
            const float v = xb[c] + __shfl_xor(xb[c], 1);  // the row's two k halves
            if (xk == 0) XBs[xr * RK + c] = v;
        }
        __syncthreads();
    }
    // accumulator element e of lane l: row 8 (e / 4) + 4 kh + e % 4 of the
    // wave's 32, column lc of the tile
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int32_t row = wave * 32 + 8 * (e >> 2) + 4 * kh + (e & 3);
        const int64_t L = L0 + row;
        if (L >= P.total) continue;
        const int32_t lm = tr.member(P, row);
        float* yrow = P.y + tr.offset(P, row, P.y_stride, P.y_plane) + o0;
        float xr_[RK];
#pragma unroll
        for (int c = 0; c < RK; ++c) xr_[c] = noisy ? XBs[row * RK + c] : 0.0f;
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const int32_t col = 32 * j + lc;
            if (col >= ct) continue;
            float yv = acc[j][e];
            if (noisy) {
                const float* ar = As + ((size_t)lm * BN + col) * RK;
                float z = 0.0f;
#pragma unroll
                for (int c = 0; c < RK; ++c) z = __fadd_rn(z, __fmul_rn(xr_[c], ar[c]));
                yv = __fadd_rn(yv, z);
            }
            yrow[col] = yv;
        }
    }
}

static int32_t f32_bn(int32_t a) { return a <= 32 ? 32 : a <= 64 ? 64 : 128; }
static int32_t f32_rk(int32_t r) { return r <= 1 ? 1 : r <= 4 ? 4 : r <= 8 ? 8 : 16; }

// Most members a 128-row tile (starting at a multiple of 128) can touch.
static int32_t f32_nm_max(int32_t R, int32_t n) {
    int32_t nm;
    if (R % KF_BM == 0) nm = 1;
    else if (R > KF_BM) nm = 2;
    else if (KF_BM % R == 0) nm = KF_BM / R;
    else nm = (KF_BM - 1) / R + 2;
    return std::min(nm, n);
}

// Rows per generating thread: up to 32 normals, fewer while that leaves under
// 64k threads; at least enough for the jump tables' row count.
static bool factor_rows(const LinParams& P, int32_t* rc_out, int32_t* groups) {
    const int32_t r = P.r, rows = P.a + P.b;
    int32_t rc = std::max(1, 32 / r);
    while (rc > 1 && (int64_t)P.n * ((rows + rc - 1) / rc) < 65536) rc = std::max(1, rc / 2);
    rc = std::max<int32_t>(rc, (int32_t)((rows + kJumpMaxRows - 1) / kJumpMaxRows));
    if ((int64_t)rc * r > kJumpMaxL) return false;
    *rc_out = rc;
    *groups = (rows + rc - 1) / rc;
    return true;
}

// The tiling of one call (shape only).
struct F32Plan {
    int32_t bn, rk, nm, bch;
    size_t lds, f_bytes;
};

static bool f32_plan(const LinParams& P, F32Plan* pl) {
    if (P.math != HSES_MATH_F32 || P.tmm || P.r > KF_RMAX || P.r < 0) return false;
    const int32_t r = P.r;
    pl->bn = f32_bn(P.a);
    pl->rk = f32_rk(r);
    pl->nm = f32_nm_max(P.R, P.n);
    const size_t bch = r > 0 ? (size_t)pl->nm * KF_BK * pl->rk : 0;
    if (bch > 8 * KF_THREADS) return false;  // BPT values per thread
    pl->bch = (int32_t)bch;
    const size_t a_lds = r > 0 ? (size_t)pl->nm * pl->bn * pl->rk : 0;
    if (a_lds > KF_AMAX) return false;
    const size_t nbuf = P.b > KF_BK ? 2 : 1;  // staging buffers (k_gemm_f32)
    pl->lds = (nbuf * ((size_t)(KF_BM + pl->bn) * KF_XP + bch) + a_lds) * 4;
    pl->f_bytes = 0;
    if (r > 0) {
        int32_t rc, groups;
        if (!factor_rows(P, &rc, &groups)) return false;
        pl->f_bytes = align16((size_t)P.n * (P.a + P.b) * r * 4);
    }
    return true;
}

int launch_factors(LinParams& P, DeviceState* st, hipStream_t s, float* F) {
    int32_t rc, groups;
    if (P.r < 1 || !factor_rows(P, &rc, &groups)) return HSES_ERR_UNSUPPORTED;
    int e = get_jump_table(st, (int64_t)rc * P.r, groups, &P.jump);
    if (e) return e;
    const int64_t blocks = ((int64_t)P.n * groups + 255) / 256;
    if (blocks > INT32_MAX) return set_error(HSES_ERR_INVALID_ARG, "too many factor rows");
    hipLaunchKernelGGL(k_factors, dim3((uint32_t)blocks), dim3(256), 0, s, P, rc, groups, F);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

size_t linear_f32_workspace(int32_t a, int32_t b, int32_t r, int32_t n, int32_t rows_per_member,
                            int32_t n_time, int32_t math) {
    (void)rows_per_member;
    (void)n_time;
    if (math != HSES_MATH_F32 || a < 1 || b < 1 || n < 1 || r < 0 || r > KF_RMAX) return 0;
    return align16((size_t)n * (a + b) * r * 4);
}

template <int XFMT, int NT>
static int launch_gemm_rk(const LinParams& P, const F32Plan& pl, hipStream_t s, const float* F,
                          dim3 grid) {
    auto launch = [&](auto kern) -> int {
        if (pl.lds > 64 * 1024)
            HSES_CHECK_HIP(hipFuncSetAttribute((const void*)kern,
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)pl.lds));
        hipLaunchKernelGGL(kern, grid, dim3(KF_THREADS), pl.lds, s, P, F, pl.bch);
        HSES_CHECK_HIP(hipGetLastError());
        return HSES_OK;
    };
    switch (pl.rk) {
        case 1: return launch(k_gemm_f32<XFMT, NT, 1>);
        case 4: return launch(k_gemm_f32<XFMT, NT, 4>);
        case 8: return launch(k_gemm_f32<XFMT, NT, 8>);
        default: return launch(k_gemm_f32<XFMT, NT, 16>);
    }
}

template <int XFMT>
static int launch_gemm_bn(const LinParams& P, const F32Plan& pl, hipStream_t s, const float* F,
                          dim3 grid) {
    switch (pl.bn) {
        case 32: return launch_gemm_rk<XFMT, 1>(P, pl, s, F, grid);
        case 64: return launch_gemm_rk<XFMT, 2>(P, pl, s, F, grid);
        default: return launch_gemm_rk<XFMT, 4>(P, pl, s, F, grid);
    }
}

int launch_linear_f32(LinParams& P, DeviceState* st, hipStream_t s, void* work, size_t work_bytes) {
    F32Plan pl;
    if (!f32_plan(P, &pl)) return HSES_ERR_UNSUPPORTED;
    if (pl.lds > st->max_lds) return HSES_ERR_UNSUPPORTED;
    if (P.r > 0 && (!work || work_bytes < pl.f_bytes)) return HSES_ERR_UNSUPPORTED;
    const int64_t row_tiles = (P.total + KF_BM - 1) / KF_BM;
    const int64_t tiles = row_tiles * ((P.a + pl.bn - 1) / pl.bn);
    if (tiles > INT32_MAX) return set_error(HSES_ERR_INVALID_ARG, "too many output rows");
    float* F = static_cast<float*>(work);
    if (P.r > 0) {
        const int rc = launch_factors(P, st, s, F);
        if (rc) return rc;
    }
    const dim3 grid((uint32_t)tiles);
    switch (P.x_fmt) {
        case HSES_FMT_BITS: return launch_gemm_bn<HSES_FMT_BITS>(P, pl, s, F, grid);
        case HSES_FMT_BF16: return launch_gemm_bn<HSES_FMT_BF16>(P, pl, s, F, grid);
        default: return launch_gemm_bn<HSES_FMT_F32>(P, pl, s, F, grid);
    }
}

}  // namespace hses
