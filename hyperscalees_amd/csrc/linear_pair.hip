// linear_pair.hip -- perturbed forward for large ranks (r = 16..128, bf16 MFMA).
//
// Reference: lora_linear_batched (burn_impl/hyperscalees-models/src/snn.rs:665-685),
// do_mm_impl (burn_impl/hyperscalees-noiser/src/eggroll.rs:419-446).
//
// At r = 128 the "low-rank" term x B_m is as large as the base product, so
// the two are one GEMM against [W^T | B_pair] and the pair's factors are the
// unit of reuse: members 2p and 2p+1 share B and use +A / -A
// (eggroll.rs:60-65).  A persistent workgroup takes pair after pair:
//   1. generates A_pair (a x r) into LDS and B_pair (b x r) into its own
//      staging slot of the caller's workspace (bf16, k-contiguous per rank
//      column; 200 KB at b = 784, more than LDS holds), each factor row by
//      one thread continuing its row of the stream;
//   2. for each 256-row block of the pair's rows: C = X [W^T | B] with
//      bf16 MFMA (8 waves as 4 row groups x {base, xB}); binary activations
//      arrive bit-packed and are expanded in LDS;
//   3. epilogue: y = base + (sign_m xB) A^T with a second MFMA over K = r,
//      stored as fp32.
// The (n, b, r) factor tensor is never materialised: at most one B per
// workgroup exists at any time.
#include <math.h>

#include "linear_common.h"
#include "mfma.h"
#include "noise_dev.h"
#include "runtime.h"

namespace hses {

constexpr int K2_THREADS = 512, K2_RB = 256, K2_BK = 32, K2_AMAX = 128, K2_RMAX = 128;
constexpr int K2_XP = K2_BK + 8;  // bf16 tile pitch (elements)

struct K2Layout {
    size_t off_a, off_xbits, off_x, off_w, off_b, off_xb, bytes;
    int32_t apitch, xbpitch, words;
    __host__ __device__ K2Layout(int r, int b) {
        // the second product steps K (= r) by 32: pad rows to a multiple of 32
        apitch = (r + 31) / 32 * 32 + 8;
        xbpitch = apitch;
        words = (b + 63) / 64;
        size_t o = align16(sizeof(BmTables));
        off_a = o;
        o = align16(o + (size_t)K2_AMAX * apitch * 2);
        const size_t stage0 = o;
        off_xbits = o;
        o = align16(o + (size_t)K2_RB * words * 8);
        off_x = o;
        o = align16(o + (size_t)K2_RB * K2_XP * 2);
        off_w = o;
        o = align16(o + (size_t)K2_AMAX * K2_XP * 2);
        off_b = o;
        o = align16(o + (size_t)K2_RMAX * K2_XP * 2);
        off_xb = stage0;  // xB staging reuses the K-loop buffers
        const size_t xb_end = align16(stage0 + (size_t)K2_RB * xbpitch * 2);
        bytes = o > xb_end ? o : xb_end;
    }
};

struct K2Extra {
    uint16_t* slots;        // [grid][r][bpitch] bf16
    const uint16_t* wbf;    // W as bf16 (a, b)
    int32_t bpitch;         // k pitch of a slot (multiple of 8)
    int32_t pair_lo, n_pairs;
};

__global__ void k_w_to_bf16(const float* __restrict__ W, int64_t len, uint16_t* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < len) out[i] = f2bf(W[i]);
}

template <int XFMT>
__global__ __launch_bounds__(K2_THREADS) void k_linear_pair(LinParams P, K2Extra E) {
    extern __shared__ __align__(16) unsigned char smem[];
    const K2Layout lay(P.r, P.b);
    BmTables* tabs = reinterpret_cast<BmTables*>(smem);
    uint16_t* As = reinterpret_cast<uint16_t*>(smem + lay.off_a);
    uint64_t* Xbits = reinterpret_cast<uint64_t*>(smem + lay.off_xbits);
    uint16_t* Xs = reinterpret_cast<uint16_t*>(smem + lay.off_x);
    uint16_t* Ws = reinterpret_cast<uint16_t*>(smem + lay.off_w);
    uint16_t* Bts = reinterpret_cast<uint16_t*>(smem + lay.off_b);
    uint16_t* XBs = reinterpret_cast<uint16_t*>(smem + lay.off_xb);

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int li = lane & 15, kg = lane >> 4;
    const int32_t r = P.r, a = P.a, b = P.b, R = P.R;
    uint16_t* slot = E.slots + (size_t)blockIdx.x * r * E.bpitch;
    const int wr = wave >> 1;        // row group: rows [64*wr, 64*wr+64) of the block
    const int wc = wave & 1;         // 0: base columns (x W^T), 1: xB columns
    const int ncols = wc == 0 ? a : r;
    const int ntile = (ncols + 15) / 16;

    load_bm_tables(tabs, P.tables);
    __syncthreads();
    const NoiseCtx ctx{tabs, P.log_exc, P.cos_exc};

    for (int32_t pi = blockIdx.x; pi < E.n_pairs; pi += gridDim.x) {
        const int32_t pair = E.pair_lo + pi;
        // Members of this pair inside the launch: m_lo .. m_hi (local indices).
        const int32_t m_even = 2 * pair - P.tid_lo;
        const int32_t m_lo = max(m_even, 0), m_hi = min(m_even + 1, P.n - 1);
        const int64_t row_lo = (int64_t)m_lo * R, row_hi = (int64_t)(m_hi + 1) * R;

        // ---- 1. factors: A rows -> LDS (bf16, [o][c]); B rows -> slot ([c][k]) ----
        {
            int32_t te, tt;
            float sg;
            epoch_thread_sign(P.epoch, 2 * pair, P.nreuse, &te, &tt, &sg);
            const uint64_t seed = noise_seed(P.key, te, tt);
            for (int32_t j = tid; j < a + b; j += K2_THREADS) {
                uint64_t s = row_start_state(seed, j, P.jump);
                if (j < b) {
                    bm_run(s, r, ctx, [&](int32_t c, float v) { slot[(size_t)c * E.bpitch + j] = f2bf(v); });
                } else {
                    uint16_t* dst = As + (size_t)(j - b) * lay.apitch;
                    bm_run(s, r, ctx, [&](int32_t c, float v) { dst[c] = f2bf(v * P.bs); });
                    for (int32_t c = r; c < ((r + 31) & ~31); ++c) dst[c] = 0;
                }
            }
            // zero the k-padding of the slot so the last K tile reads zeros
            for (int32_t i = tid; i < r * (E.bpitch - b); i += K2_THREADS) {
                const int32_t c = i / (E.bpitch - b), k = b + i % (E.bpitch - b);
                slot[(size_t)c * E.bpitch + k] = 0;
            }
            __threadfence_block();
            __syncthreads();
        }

        // ---- 2./3. row blocks ----------------------------------------------------
        for (int64_t L0 = row_lo; L0 < row_hi; L0 += K2_RB) {
            f32x4 acc[4][8];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0, 0, 0, 0};

            if constexpr (XFMT == HSES_FMT_BITS) {
                // Whole bit rows of the block into LDS once.
                for (int32_t i = tid; i < K2_RB * lay.words; i += K2_THREADS) {
                    const int32_t row = i / lay.words, w = i % lay.words;
                    const int64_t Lr = L0 + row;
                    Xbits[i] = Lr < row_hi
                                   ? static_cast<const uint64_t*>(P.x)[phys_row(P, Lr, P.x_stride, P.x_plane) + w]
                                   : 0ull;
                }
                __syncthreads();
            }
            const int srow = tid >> 1, sk = (tid & 1) * 16;  // x staging: 256 rows x 2 x 16
            const int64_t Ls = L0 + srow;
            const bool svalid = Ls < row_hi;
            const int64_t xoff = (XFMT != HSES_FMT_BITS && svalid) ? phys_row(P, Ls, P.x_stride, P.x_plane) : 0;

            for (int32_t k0 = 0; k0 < b; k0 += K2_BK) {
                // x tile (256 x 32) as bf16
                if constexpr (XFMT == HSES_FMT_BITS) {
                    const int32_t k = k0 + sk;
                    uint32_t bits = (uint32_t)(Xbits[srow * lay.words + (k >> 6)] >> (k & 63)) & 0xffffu;
                    if (b - k < 16) bits &= b - k > 0 ? (1u << (b - k)) - 1u : 0u;
                    u16x8 v0, v1;
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        v0[i] = ((bits >> i) & 1u) ? (uint16_t)0x3f80 : (uint16_t)0;
                        v1[i] = ((bits >> (i + 8)) & 1u) ? (uint16_t)0x3f80 : (uint16_t)0;
                    }
                    *reinterpret_cast<u16x8*>(&Xs[srow * K2_XP + sk]) = v0;
                    *reinterpret_cast<u16x8*>(&Xs[srow * K2_XP + sk + 8]) = v1;
                } else {
                    uint16_t v[16];
                    load_x_seg<HSES_MATH_BF16, XFMT>(P.x, xoff, svalid, k0 + sk, b, v);
                    load_x_seg<HSES_MATH_BF16, XFMT>(P.x, xoff, svalid, k0 + sk + 8, b, v + 8);
#pragma unroll
                    for (int i = 0; i < 16; ++i) Xs[srow * K2_XP + sk + i] = v[i];
                }
                // W tile (a x 32) and B tile (r x 32), 8 elements per thread
                for (int32_t i = tid; i < (K2_AMAX + K2_RMAX) * 4; i += K2_THREADS) {
                    const int32_t row = i >> 2, seg = (i & 3) * 8;
                    u16x8 v = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
                    if (row < K2_AMAX) {
                        if (row < a) {
                            const uint16_t* src = E.wbf + (size_t)row * b + k0 + seg;
#pragma unroll
                            for (int e = 0; e < 8; ++e) v[e] = (k0 + seg + e < b) ? src[e] : (uint16_t)0;
                        }
                        *reinterpret_cast<u16x8*>(&Ws[row * K2_XP + seg]) = v;
                    } else {
                        const int32_t c = row - K2_AMAX;
                        if (c < r) v = *reinterpret_cast<const u16x8*>(slot + (size_t)c * E.bpitch + k0 + seg);
                        *reinterpret_cast<u16x8*>(&Bts[c * K2_XP + seg]) = v;
                    }
                }
                __syncthreads();
                const uint16_t* Bop = wc == 0 ? Ws : Bts;
                u16x8 af[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) af[i] = lds_u16x8(&Xs[(wr * 64 + i * 16 + li) * K2_XP + kg * 8]);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    if (j >= ntile) break;
                    const u16x8 bf = lds_u16x8(&Bop[(j * 16 + li) * K2_XP + kg * 8]);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[i][j] = mfma_bf16(af[i], bf, acc[i][j]);
                }
                __syncthreads();
            }

            // xB waves: sign_m * xB -> LDS as bf16 [row][c]
            if (wc == 1) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int row = wr * 64 + i * 16 + 4 * kg + v;
                        const int64_t Lr = L0 + row;
                        const int32_t m = (int32_t)(Lr / R);
                        const float sgn = ((P.tid_lo + m) & 1) ? -1.0f : 1.0f;
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            if (j < ntile)
                                XBs[row * lay.xbpitch + j * 16 + li] = f2bf(sgn * acc[i][j][v]);
                            else if (j * 16 < ((r + 31) & ~31))
                                XBs[row * lay.xbpitch + j * 16 + li] = 0;  // K tail of the 2nd product
                        }
                    }
            }
            __syncthreads();
            // base waves: acc += (sign xB) A^T  (K = r), then store y
            if (wc == 0) {
                for (int32_t c0 = 0; c0 < r; c0 += 32) {
                    u16x8 xf[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) xf[i] = lds_u16x8(&XBs[(wr * 64 + i * 16 + li) * lay.xbpitch + c0 + kg * 8]);
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        if (j >= ntile) break;
                        const u16x8 af2 = lds_u16x8(&As[(j * 16 + li) * lay.apitch + c0 + kg * 8]);
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[i][j] = mfma_bf16(xf[i], af2, acc[i][j]);
                    }
                }
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int row = wr * 64 + i * 16 + 4 * kg + v;
                        const int64_t Lr = L0 + row;
                        if (Lr >= row_hi) continue;
                        float* yrow = P.y + phys_row(P, Lr, P.y_stride, P.y_plane);
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            const int col = j * 16 + li;
                            if (j < ntile && col < a) yrow[col] = acc[i][j][v];
                        }
                    }
            }
            __syncthreads();
        }
    }
}

static bool pair_kernel_applies(const LinParams& P) {
    return P.math == HSES_MATH_BF16 && P.r >= 16 && P.r <= K2_RMAX && P.r % 16 == 0 &&
           P.a <= K2_AMAX;
}

static int32_t pair_grid(const DeviceState* st, int32_t n_pairs) {
    return std::max(1, std::min(n_pairs, st->num_cus));
}

static void pair_range(int32_t tid_lo, int32_t n, int32_t* lo, int32_t* cnt) {
    *lo = tid_lo / 2;
    *cnt = (tid_lo + n - 1) / 2 - *lo + 1;
}

size_t linear_pair_workspace(const DeviceState* st, int32_t a, int32_t b, int32_t r, int32_t n) {
    int32_t lo, cnt;
    pair_range(0, n, &lo, &cnt);
    const int32_t grid = pair_grid(st, cnt + 1);
    const int32_t bpitch = (b + K2_BK - 1) / K2_BK * K2_BK + 8;
    return align16((size_t)a * b * 2) + (size_t)grid * r * bpitch * 2;
}

int launch_linear_pair(LinParams& P, DeviceState* st, hipStream_t s, void* work, size_t work_bytes) {
    if (P.r == 0 || !pair_kernel_applies(P)) return HSES_ERR_UNSUPPORTED;
    const K2Layout lay(P.r, P.b);
    if (lay.bytes > st->max_lds) return HSES_ERR_UNSUPPORTED;
    K2Extra E{};
    pair_range(P.tid_lo, P.n, &E.pair_lo, &E.n_pairs);
    E.bpitch = (P.b + K2_BK - 1) / K2_BK * K2_BK + 8;
    const int32_t grid = pair_grid(st, E.n_pairs);
    const size_t need = align16((size_t)P.a * P.b * 2) + (size_t)grid * P.r * E.bpitch * 2;
    if (!work || work_bytes < need)
        return set_error(HSES_ERR_INVALID_ARG, "hses_perturbed_linear: workspace too small");
    uint16_t* wbf = static_cast<uint16_t*>(work);
    E.wbf = wbf;
    E.slots = reinterpret_cast<uint16_t*>(static_cast<char*>(work) + align16((size_t)P.a * P.b * 2));
    int rc = get_jump_table(st, P.r, (int64_t)P.a + P.b, &P.jump);
    if (rc) return rc;
    const int64_t wl = (int64_t)P.a * P.b;
    hipLaunchKernelGGL(k_w_to_bf16, dim3((uint32_t)((wl + 255) / 256)), dim3(256), 0, s, P.W, wl, wbf);
    HSES_CHECK_HIP(hipGetLastError());
    auto launch = [&](auto kern) -> int {
        if (lay.bytes > 64 * 1024)
            HSES_CHECK_HIP(hipFuncSetAttribute((const void*)kern,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lay.bytes));
        hipLaunchKernelGGL(kern, dim3(grid), dim3(K2_THREADS), lay.bytes, s, P, E);
        HSES_CHECK_HIP(hipGetLastError());
        return HSES_OK;
    };
    switch (P.x_fmt) {
        case HSES_FMT_F32: return launch(k_linear_pair<HSES_FMT_F32>);
        case HSES_FMT_BF16: return launch(k_linear_pair<HSES_FMT_BF16>);
        default: return launch(k_linear_pair<HSES_FMT_BITS>);
    }
}

}  // namespace hses
