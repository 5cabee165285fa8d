// linear_wide.hip -- the batched EggRoll perturbed forward for wide outputs at
// small rank, on bf16 MFMA:
//   do_mm  (eggroll.rs:419-446):  y = x W^T + (x B_m) A_m^T,
//   do_Tmm (eggroll.rs:450-477):  y = x W + (x A_m) B_m^T,
// with an optional elementwise activation fused into the epilogue and an fp32
// or bf16 output.
//
// A workgroup of 8 waves owns a 128-row tile of the output and sweeps its
// 256-column tiles (64 or 128 for outputs that narrow) (rows are member-major, a row tile touches at most a few
// members; their noise columns, nm * r <= 16, ride along as one extra
// 16-wide operand):
//   1. W is converted once per call to bf16 (a, kp) in the workspace; the
//      row tile's members' input-side factors (K x r each) and output-side
//      factors (a x r each) are generated once from the noiser stream into LDS;
//   2. one pipeline over (column tile, K step of 64): x (fp32, bf16 or
//      bit-packed) and W tiles are prefetched into registers one step ahead,
//      also across column tiles, stored to LDS as bf16, and each wave
//      accumulates its 64 x 64 sub-tile with 32x32x16 MFMAs (fp32
//      accumulation); during the first column tile each wave also forms a
//      16-row slice of x B_m with 16x16x32 MFMAs;
//   3. after a column tile's last K step: y = acc + (x B_m) A_m^T (r
//      multiply-adds), activation, store, and the accumulators restart.
#include <math.h>

#include <type_traits>

#include "linear_common.h"
#include "mfma.h"
#include "noise_dev.h"
#include "runtime.h"
#include "tile_factors.h"

namespace hses {

constexpr int KW_BM = 128, KW_BN = 256, KW_BK = 64, KW_THREADS = 512;  // KW_BN: widest pass
constexpr int KW_XP = KW_BK + 8;  // LDS pitch of the x and W tiles (bf16 elements, 144 B)
constexpr int KW_NE = 16;         // noise columns (members x rank) per tile

typedef float f32x16w __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16w mfma32w(const u16x8& a, const u16x8& b, f32x16w c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

struct KWLayout {
    size_t off_x, off_w, off_b, off_a, off_xb, bytes;
    __host__ __device__ KWLayout(int ne_real, int bpitch, int nm_max, int r, int a, bool noisy) {
        size_t o = noisy ? align16(sizeof(BmTables)) : 0;
        off_x = o;
        o = align16(o + (size_t)KW_BM * KW_XP * 2);
        off_w = o;
        o = align16(o + (size_t)KW_BN * KW_XP * 2);
        off_b = o;
        o = align16(o + (size_t)ne_real * bpitch * 2);
        off_a = o;
        o = align16(o + (noisy ? (size_t)nm_max * a * r * 4 : 0));
        off_xb = o;
        o = align16(o + (noisy ? (size_t)KW_BM * KW_NE * 4 : 0));
        bytes = o;
    }
};

template <int ACT>
__device__ __forceinline__ float act_apply(float v) {
    if constexpr (ACT == ACT_TANH) return tanhf(v);
    if constexpr (ACT == ACT_SIGMOID) return 1.0f / (1.0f + expf(-v));
    if constexpr (ACT == ACT_RELU_SQ) {
        const float z = v > 0.0f ? v : 0.0f;
        return z * z;
    }
    return v;
}

// BN: columns per pass (256, or 128 / 64 for narrow outputs).  The 8 waves
// form WR x WC (rows x columns); each wave owns WI x WJ blocks of 32 x 32.
template <int XFMT, int ACT, bool YBF16, int BN>
__global__ __launch_bounds__(KW_THREADS, 4) void k_linear_wide(LinParams P, const uint16_t* __restrict__ Wb,
                                                            int32_t kp, int32_t col_tiles) {
    extern __shared__ __align__(16) unsigned char smem[];
    const bool noisy = P.ne_real > 0;
    const KWLayout lay(P.ne_real, P.bpitch, P.nm_max, P.r, P.a, noisy);
    BmTables* tabs = reinterpret_cast<BmTables*>(smem);
    uint16_t* Xs = reinterpret_cast<uint16_t*>(smem + lay.off_x);
    uint16_t* Ws = reinterpret_cast<uint16_t*>(smem + lay.off_w);
    uint16_t* Bs = reinterpret_cast<uint16_t*>(smem + lay.off_b);
    float* As = reinterpret_cast<float*>(smem + lay.off_a);
    float* XB = reinterpret_cast<float*>(smem + lay.off_xb);

    const int64_t L0 = (int64_t)blockIdx.x * KW_BM;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    constexpr int WC = BN == 256 ? 4 : 2, WR = 8 / WC;
    constexpr int WI = KW_BM / (32 * WR), WJ = BN / (32 * WC);
    constexpr int WROWS = KW_BM / WR, WCOLS = BN / WC;
    constexpr int NW = BN / 64;  // W uint4 loads per thread per K step
    const int wr = wave / WC, wc = wave % WC, lc = lane & 31, hl = lane >> 5;
    const int32_t b = P.b, R = P.R, a = P.a;
    const int32_t nkt = (b + KW_BK - 1) / KW_BK;
    const bool flat = P.n_time == 1;  // physical row = logical row
    const int32_t m_first = (int32_t)(L0 / R);
    const int32_t m_last = (int32_t)((min(L0 + KW_BM, P.total) - 1) / R);

    // ---- staging: x rows and W columns this thread loads ----------------------
    // F32: 4 rows (step 32) x 4 k; BF16: 2 rows (step 64) x 8 k; BITS (threads
    // below 256): one row, 32 k (half of the row's 64-bit word of this K step).
    constexpr bool BITS = XFMT == HSES_FMT_BITS;
    constexpr int XR = XFMT == HSES_FMT_F32 ? 4 : (BITS ? 1 : 2);
    constexpr int XSTEP = XFMT == HSES_FMT_F32 ? 32 : 64;
    const int xseg = XFMT == HSES_FMT_F32 ? (tid & 15) * 4 : (BITS ? (tid & 1) * 32 : (tid & 7) * 8);
    const int xrow0 = XFMT == HSES_FMT_F32 ? tid >> 4 : (BITS ? (tid & 255) >> 1 : tid >> 3);
    const bool xload = !BITS || tid < 2 * KW_BM;
    int64_t xoff[XR];
#pragma unroll
    for (int i = 0; i < XR; ++i) {
        const int64_t Lr = L0 + xrow0 + XSTEP * i;
        xoff[i] = (xload && Lr < P.total) ? (flat ? Lr * P.x_stride : phys_row(P, Lr, P.x_stride, P.x_plane)) : -1;
    }
    const int wseg = (tid & 7) * 8, wcol0 = tid >> 3;  // W: NW columns (step 64) x 8 k
    uint4 xr_[XR];
    uint32_t xbits = 0;
    uint4 wr_[NW];

    auto load_tiles = [&](int32_t ct_i, int32_t kt) {
        const int32_t k = kt * KW_BK + xseg;
        if constexpr (BITS) {
            // bits past column b are masked off (the ABI does not require them zero)
            const int32_t nb = min(max(b - k, 0), 32);
            const uint32_t mask = nb >= 32 ? 0xffffffffu : (1u << nb) - 1u;
            xbits = (xoff[0] >= 0 && nb > 0)
                        ? static_cast<const uint32_t*>(P.x)[2 * (xoff[0] + kt) + (xseg >> 5)] & mask
                        : 0u;
        } else if constexpr (XFMT == HSES_FMT_F32) {
            const float* xp = static_cast<const float*>(P.x);
#pragma unroll
            for (int i = 0; i < XR; ++i)
                xr_[i] = (xoff[i] >= 0 && k < b) ? *reinterpret_cast<const uint4*>(xp + xoff[i] + k)
                                                 : uint4{0, 0, 0, 0};
        } else {
            const uint16_t* xp = static_cast<const uint16_t*>(P.x);
#pragma unroll
            for (int i = 0; i < XR; ++i)
                xr_[i] = (xoff[i] >= 0 && k < b) ? *reinterpret_cast<const uint4*>(xp + xoff[i] + k)
                                                 : uint4{0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            const int32_t col = ct_i * BN + wcol0 + 64 * i;
            wr_[i] = col < a ? *reinterpret_cast<const uint4*>(Wb + (int64_t)col * kp + kt * KW_BK + wseg)
                             : uint4{0, 0, 0, 0};
        }
    };
    auto store_tiles = [&]() {
        if constexpr (BITS) {
            if (xload) {
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    *reinterpret_cast<u16x8*>(Xs + xrow0 * KW_XP + xseg + 8 * q) =
                        expand_bits((xbits >> (8 * q)) & 0xffu);
            }
        } else if constexpr (XFMT == HSES_FMT_F32) {
#pragma unroll
            for (int i = 0; i < XR; ++i) {
                const uint2 v{pack_bf16x2(__uint_as_float(xr_[i].x), __uint_as_float(xr_[i].y)),
                              pack_bf16x2(__uint_as_float(xr_[i].z), __uint_as_float(xr_[i].w))};
                *reinterpret_cast<uint2*>(Xs + (xrow0 + XSTEP * i) * KW_XP + xseg) = v;
            }
        } else {
#pragma unroll
            for (int i = 0; i < XR; ++i)
                *reinterpret_cast<uint4*>(Xs + (xrow0 + XSTEP * i) * KW_XP + xseg) = xr_[i];
        }
#pragma unroll
        for (int i = 0; i < NW; ++i)
            *reinterpret_cast<uint4*>(Ws + (wcol0 + 64 * i) * KW_XP + wseg) = wr_[i];
    };

    // ---- 1. factors of the row tile's members into LDS -------------------------
    if (noisy) {
        load_bm_tables(tabs, P.tables);
        for (int i = tid; i < P.ne_real * P.bpitch; i += KW_THREADS) Bs[i] = 0;
        __syncthreads();
        const NoiseCtx ctx{tabs, P.log_exc, P.cos_exc};
        gen_tile_factors<HSES_MATH_BF16>(P, ctx, m_first, m_last - m_first + 1, 0, a, Bs,
                                         P.bpitch, As, a);
    }

    // ---- 2. one pipeline over (column tile, K step) -----------------------------
    f32x16w acc[WI][WJ];
#pragma unroll
    for (int i = 0; i < WI; ++i)
#pragma unroll
        for (int j = 0; j < WJ; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
    f32x4 accx = f32x4{0, 0, 0, 0};
    const int xb_row = wave * 16 + (lane & 15);  // the 16 x B rows of this wave
    const int xb_e = lane & 15, xb_kg = lane >> 4;
    const bool xb_on = noisy && xb_e < P.ne_real;
    const int32_t r = P.r;

    load_tiles(0, 0);  // after the generation, whose registers it would otherwise share
    int32_t ct_i = 0, kt = 0;
    const int32_t nsteps = col_tiles * nkt;
    for (int32_t step = 0; step < nsteps; ++step) {
        store_tiles();
        __syncthreads();
        if (step + 1 < nsteps) {
            const bool same = kt + 1 < nkt;
            load_tiles(same ? ct_i : ct_i + 1, same ? kt + 1 : 0);
        }
#pragma unroll
        for (int ks = 0; ks < KW_BK / 16; ++ks) {
            const int kk = ks * 16 + hl * 8;
            u16x8 af[WI], bf[WJ];
#pragma unroll
            for (int i = 0; i < WI; ++i) af[i] = lds_u16x8(Xs + (wr * WROWS + 32 * i + lc) * KW_XP + kk);
#pragma unroll
            for (int j = 0; j < WJ; ++j) bf[j] = lds_u16x8(Ws + (wc * WCOLS + 32 * j + lc) * KW_XP + kk);
#pragma unroll
            for (int i = 0; i < WI; ++i)
#pragma unroll
                for (int j = 0; j < WJ; ++j) acc[i][j] = mfma32w(af[i], bf[j], acc[i][j]);
        }
        if (noisy && ct_i == 0) {
#pragma unroll
            for (int k32 = 0; k32 < KW_BK / 32; ++k32) {
                const int kk = k32 * 32 + xb_kg * 8;
                const u16x8 bx = xb_on ? lds_u16x8(Bs + xb_e * P.bpitch + kt * KW_BK + kk)
                                       : u16x8{0, 0, 0, 0, 0, 0, 0, 0};
                accx = mfma_bf16(lds_u16x8(Xs + xb_row * KW_XP + kk), bx, accx);
            }
        }
        __syncthreads();
        if (kt + 1 < nkt) {
            ++kt;
            continue;
        }

        // ---- 3. epilogue of column tile ct_i ---------------------------------------
        if (noisy && ct_i == 0) {
            // 16x16 layout: lane l holds D[4 (l / 16) + v][l % 16]
#pragma unroll
            for (int v = 0; v < 4; ++v) XB[(wave * 16 + 4 * xb_kg + v) * KW_NE + xb_e] = accx[v];
            __syncthreads();
        }
        const int32_t o0 = ct_i * BN;
        const int32_t ct = min(BN, a - o0);
        // The row addresses below are the same for every column tile; computing
        // them here (the empty asm hides that) keeps the compiler from holding
        // all 32 of them in registers across the whole pipeline.
        int32_t rbase = wr * WROWS + 4 * hl;
        asm volatile("" : "+v"(rbase));
#pragma unroll
        for (int i = 0; i < WI; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                // 32x32 layout: lane l holds D[8 (e / 4) + 4 (l / 32) + e % 4][l % 32]
                const int row = rbase + 32 * i + 8 * (e >> 2) + (e & 3);
                const int64_t Lr = L0 + row;
                if (Lr >= P.total) continue;
                int32_t lm = 0;
                if (noisy && P.nm_max > 1) lm = (int32_t)((Lr - (int64_t)m_first * R) / R);
                const int64_t yoff = (flat ? Lr * P.y_stride : phys_row(P, Lr, P.y_stride, P.y_plane)) + o0;
#pragma unroll
                for (int j = 0; j < WJ; ++j) {
                    const int col = wc * WCOLS + 32 * j + lc;
                    if (col >= ct) continue;
                    float v = acc[i][j][e];
                    if (noisy) {
                        const float* xb = XB + row * KW_NE + lm * r;
                        const float* ar = As + ((size_t)lm * a + o0 + col) * r;
                        float z = 0.0f;
                        for (int32_t c = 0; c < r; ++c) z = __fadd_rn(z, __fmul_rn(xb[c], ar[c]));
                        v = __fadd_rn(v, z);
                    }
                    if constexpr (YBF16)
                        reinterpret_cast<uint16_t*>(P.y)[yoff + col] = f2bf(act_apply<ACT>(v));
                    else
                        P.y[yoff + col] = act_apply<ACT>(v);
                }
            }
#pragma unroll
        for (int i = 0; i < WI; ++i)
#pragma unroll
            for (int j = 0; j < WJ; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
        ++ct_i;
        kt = 0;
    }
}

static int32_t wide_nm_max(int32_t R, int32_t n) {
    int32_t nm;
    if (R % KW_BM == 0)
        nm = 1;
    else if (KW_BM % R == 0)
        nm = KW_BM / R;
    else
        nm = (KW_BM - 1) / R + 2;
    return std::min(nm, n);
}

static int32_t wide_kp(int32_t b) { return (b + KW_BK - 1) / KW_BK * KW_BK; }

size_t linear_wide_workspace(int32_t a, int32_t b, int32_t r, int32_t n, int32_t rows_per_member,
                             int32_t n_time, int32_t math) {
    if (math != HSES_MATH_BF16 || a < 1 || b < 1 || n < 1 || r < 0) return 0;
    if ((int64_t)rows_per_member * n_time > INT32_MAX) return 0;
    if (r > 0 && wide_nm_max(rows_per_member * n_time, n) * r > KW_NE) return 0;
    return align16((size_t)a * wide_kp(b) * 2);
}

int launch_linear_wide(LinParams& P, DeviceState* st, hipStream_t s, void* work, size_t work_bytes,
                       int32_t act, int32_t y_fmt) {
    if (P.math != HSES_MATH_BF16) return HSES_ERR_UNSUPPORTED;
    if (P.x_fmt == HSES_FMT_BITS) {
        if (reinterpret_cast<uintptr_t>(P.x) % 8) return HSES_ERR_UNSUPPORTED;
    } else {
        if (P.x_fmt != HSES_FMT_F32 && P.x_fmt != HSES_FMT_BF16) return HSES_ERR_UNSUPPORTED;
        const int32_t vec = P.x_fmt == HSES_FMT_F32 ? 4 : 8;  // elements per 16-byte load
        if (P.b % vec || P.x_stride % vec || (P.n_time > 1 && P.x_plane % vec) ||
            reinterpret_cast<uintptr_t>(P.x) % 16)
            return HSES_ERR_UNSUPPORTED;
    }
    const bool noisy = P.r > 0 && P.bs != 0.0f;
    const int32_t nm_max = wide_nm_max(P.R, P.n);
    if (noisy && nm_max * P.r > KW_NE) return HSES_ERR_UNSUPPORTED;
    const int32_t kp = wide_kp(P.b);
    const size_t wbytes = align16((size_t)P.a * kp * 2);
    if (!work || work_bytes < wbytes) return HSES_ERR_UNSUPPORTED;
    P.nm_max = nm_max;
    P.ne_real = noisy ? nm_max * P.r : 0;
    P.ne = KW_NE;
    P.bpitch = kp + 8;
    // about one jump and a few normals per thread: groups of rc stream rows
    P.rc = noisy ? std::max(1, std::min(32 / P.r, (P.b + P.a) / KW_THREADS)) : 1;
    const KWLayout lay(P.ne_real, P.bpitch, nm_max, P.r, P.a, noisy);
    if (lay.bytes > st->max_lds) return HSES_ERR_UNSUPPORTED;
    if (noisy) {
        const int64_t chunks = (P.a + P.b + P.rc - 1) / P.rc;
        int rc = get_jump_table(st, (int64_t)P.rc * P.r, chunks, &P.jump);
        if (rc) return rc;
    }
    uint16_t* wb = static_cast<uint16_t*>(work);
    launch_w_to_bf16(P.W, P.a, P.b, kp, P.tmm, wb, s);
    HSES_CHECK_HIP(hipGetLastError());
    const int64_t row_tiles = (P.total + KW_BM - 1) / KW_BM;
    const int32_t bn = P.a <= 64 ? 64 : P.a <= 128 ? 128 : KW_BN;
    const int32_t col_tiles = (P.a + bn - 1) / bn;
    if (row_tiles > INT32_MAX / 2) return set_error(HSES_ERR_INVALID_ARG, "too many output rows");
    auto launch = [&](auto kern) -> int {
        if (lay.bytes > 64 * 1024)
            HSES_CHECK_HIP(hipFuncSetAttribute((const void*)kern,
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)lay.bytes));
        hipLaunchKernelGGL(kern, dim3((uint32_t)row_tiles), dim3(KW_THREADS), lay.bytes, s, P,
                           (const uint16_t*)wb, kp, col_tiles);
        HSES_CHECK_HIP(hipGetLastError());
        return HSES_OK;
    };
    const bool ybf = y_fmt == HSES_FMT_BF16;
    auto by_bn = [&](auto f, auto act_c, auto ybf_c) -> int {
        constexpr int F = decltype(f)::value, A = decltype(act_c)::value;
        constexpr bool Y = decltype(ybf_c)::value;
        if (bn == 64) return launch(k_linear_wide<F, A, Y, 64>);
        if (bn == 128) return launch(k_linear_wide<F, A, Y, 128>);
        return launch(k_linear_wide<F, A, Y, KW_BN>);
    };
    using std::integral_constant;
#define KW_CASE(F, A)                                                                         \
    if (P.x_fmt == F && act == A)                                                             \
        return ybf ? by_bn(integral_constant<int, F>{}, integral_constant<int, A>{},          \
                           integral_constant<bool, true>{})                                   \
                   : by_bn(integral_constant<int, F>{}, integral_constant<int, A>{},          \
                           integral_constant<bool, false>{});
    KW_CASE(HSES_FMT_F32, ACT_NONE)
    KW_CASE(HSES_FMT_F32, ACT_TANH)
    KW_CASE(HSES_FMT_F32, ACT_SIGMOID)
    KW_CASE(HSES_FMT_F32, ACT_RELU_SQ)
    KW_CASE(HSES_FMT_BF16, ACT_NONE)
    KW_CASE(HSES_FMT_BF16, ACT_TANH)
    KW_CASE(HSES_FMT_BF16, ACT_SIGMOID)
    KW_CASE(HSES_FMT_BF16, ACT_RELU_SQ)
#undef KW_CASE
    if (P.x_fmt == HSES_FMT_BITS && act == ACT_NONE && !ybf)
        return by_bn(integral_constant<int, HSES_FMT_BITS>{}, integral_constant<int, ACT_NONE>{},
                     integral_constant<bool, false>{});
    if (P.x_fmt == HSES_FMT_BITS) return HSES_ERR_UNSUPPORTED;  // other forms: unfused path
    return set_error(HSES_ERR_INVALID_ARG, "unknown activation");
}

}  // namespace hses
