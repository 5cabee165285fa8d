// linear_bf16.hip -- bf16 perturbed forward for outputs at least 256 wide at
// ranks up to 4:
//   do_mm  (eggroll.rs:419-446):  y = x W^T + (x B_m) A_m^T,
//   do_Tmm (eggroll.rs:450-477):  y = x W + (x A_m) B_m^T,
// with an optional elementwise activation and an fp32 or bf16 output (the
// Linear / Tmm layers of the RWKV-7 LM, llm.rs:182-480).
//
// After W is converted once per call to bf16 (output rows x kp, transposed for
// do_Tmm) and k_factors has drawn every member's factor rows:
//   k_gemm_bf16: a 256 x 256 output tile per workgroup; 8 waves of 64 rows x
//   128 columns on bf16 MFMA 32x32x16 with fp32 accumulation.  K runs in steps
//   of 64, double-buffered in LDS: right after a step's barrier every thread
//   issues the next step's x and W loads into registers, the waves run the
//   step's MFMAs, and the registers go to the other buffer before the next
//   barrier.  Each thread also accumulates x B_m for its row and 32-column
//   half of the step on the vector ALU (x as staged, the input-side factor
//   rounded to bf16, fp32 sums); the epilogue adds (x B_m) A_m^T with the
//   output-side factor in fp32, applies the activation and stores.
// Tiles are ordered so that each XCD (workgroups are dealt to the 8 in turn)
// works through a contiguous range with the column tiles of a row tile
// adjacent: the workgroups reading one x row tile share an L2.
#include <math.h>

#include <type_traits>

#include "linear_common.h"
#include "mfma.h"
#include "runtime.h"

namespace hses {

constexpr int KB_BM = 256, KB_BN = 256, KB_BK = 64, KB_THREADS = 512;
constexpr int KB_P = KB_BK + 8;        // LDS pitch of an x / W row (bf16): 144 B
constexpr int KB_BUF = KB_BM * KB_P;   // bf16 elements of one x (or W) buffer
constexpr int KB_RMAX = 4;
constexpr int KB_BPT = 2;              // input-side factor values staged per thread and step

// The direct-to-LDS pipeline (bf16 x, K a multiple of 64): K steps of 64 in
// two LDS stages, the next step's loads in flight during a step.  A stage holds
// x and W as 8-row blocks of 1 KB: row r of a block at r * 128 bytes, its k
// chunk c (8 bf16) in slot c ^ r, so one global_load_lds_dwordx4 fills a block
// from eight whole 128-byte rows (lane p: row p / 8, chunk (p % 8) ^ (p / 8))
// and the MFMA operand reads of eight lanes (eight rows, one chunk) hit
// distinct banks.  Then the input-side factor values of the step (fp32,
// [member][64 k], one more load).
constexpr int DL_BK = 64, DL_NS = 2;
constexpr int DL_XB = KB_BM * DL_BK * 2;          // bytes of x per stage
constexpr int DL_WB = KB_BN * DL_BK * 2;          // bytes of W per stage
constexpr int DL_FB = 1024;                       // bytes of factor values per stage
constexpr int DL_SB = DL_XB + DL_WB + DL_FB;      // 66560 bytes per stage

typedef float f32x16b __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x2b __attribute__((ext_vector_type(2)));

// a.lo b.lo + a.hi b.hi + c for bf16 pairs (v_dot2c_f32_bf16)
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2b, a), __builtin_bit_cast(bf16x2b, b),
                                           c, false);
}

__device__ __forceinline__ f32x16b mfma32b(const u16x8& a, const u16x8& b, f32x16b c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

template <int ACT>
__device__ __forceinline__ float act_value(float v) {
    if constexpr (ACT == ACT_TANH) return tanhf(v);
    if constexpr (ACT == ACT_SIGMOID) return 1.0f / (1.0f + expf(-v));
    if constexpr (ACT == ACT_RELU_SQ) {
        const float z = v > 0.0f ? v : 0.0f;
        return z * z;
    }
    return v;
}

// 32 bytes of a pipeline stage's factor values (two 16-byte LDS reads and
// their wait).  LDS reads the compiler does not see: it would otherwise wait
// for every stage load in flight (it cannot tell the stages apart); the
// stage's own loads are complete by the pipeline's explicit vmcnt wait and
// barrier.
__device__ __forceinline__ void lds_f8_dl(const float* p, float4& lo, float4& hi) {
    asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %2 offset:16\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(lo), "=&v"(hi)
                 : "v"((uint32_t)reinterpret_cast<uintptr_t>(p))
                 : "memory");
}

// s_waitcnt vmcnt(N) (expcnt and lgkmcnt not waited for), gfx9 encoding
template <int N>
__device__ __forceinline__ void vm_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// RK: rank padded to 1 or 4 (zeros past r).  bch: words of one step's staged
// input-side factor rows, as bf16 pairs of consecutive k ([lm][32][RK], 0
// without noise).  DL: the direct-to-LDS pipeline (bf16 x, rank
// 0 or 1, b % 64 == 0); otherwise x and W go through registers, one 64-wide
// step ahead.
template <int XFMT, int RK, bool DL>
__global__ __launch_bounds__(KB_THREADS) void k_gemm_bf16(LinParams P, const uint16_t* __restrict__ Wb,
                                                          int32_t kp, const float* __restrict__ F,
                                                          int32_t bch, int32_t act, int32_t ybf16,
                                                          int32_t vec_y) {
    static_assert(!DL || XFMT == HSES_FMT_BF16, "the direct-to-LDS pipeline takes bf16 x");
    extern __shared__ __align__(16) unsigned char smem[];
    uint16_t* Xs = reinterpret_cast<uint16_t*>(smem);   // [2][256][KB_P]; DL: [DL_NS][DL_SB] bytes
    uint16_t* Ws = Xs + 2 * KB_BUF;                      // [2][256][KB_P]
    uint32_t* Bc = reinterpret_cast<uint32_t*>(Ws + 2 * KB_BUF);  // [2][bch] bf16 pairs
    float* As = DL ? reinterpret_cast<float*>(smem + DL_NS * DL_SB)
                   : reinterpret_cast<float*>(Bc + 2 * bch);  // [lm][256][RK]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lc = lane & 31, hl = lane >> 5;
    const int wr = wave >> 1, wc = wave & 1;  // wave tile: rows 64 wr.., columns 128 wc..
    int64_t L0;
    int32_t o0;
    {
        const uint32_t nb = gridDim.x, g = blockIdx.x, xcd = g & 7u, j = g >> 3;
        const uint32_t q = nb >> 3, rem = nb & 7u;
        const uint32_t ncol = (uint32_t)((P.a + KB_BN - 1) / KB_BN);
        const uint32_t t = ncol == 1 ? g
                           : xcd < rem ? xcd * (q + 1) + j : rem * (q + 1) + (xcd - rem) * q + j;
        L0 = (int64_t)(t / ncol) * KB_BM;
        o0 = (int32_t)(t % ncol) * KB_BN;
    }
    const int32_t a = P.a, b = P.b, r = P.r;
    const int32_t rows_here = (int32_t)min<int64_t>(KB_BM, P.total - L0);
    const TileRows tr(P, L0);
    const int32_t nm = tr.member(P, rows_here - 1) + 1;
    const bool noisy = r > 0;
    const int64_t fpitch = (int64_t)(a + b) * r;
    const float* Fm = F + (int64_t)tr.m_first * fpitch;
    const int32_t in_off = P.tmm ? a : 0, out_off = P.tmm ? 0 : b;  // factor rows by role

    // ---- output-side factor rows of the tile's columns (fp32) ------------------
    if (noisy) {
        for (int32_t i = tid; i < nm * KB_BN * RK; i += KB_THREADS) {
            const int32_t c = i % RK, o = (i / RK) % KB_BN, lm = i / (RK * KB_BN);
            As[i] = (c < r && o0 + o < a) ? Fm[lm * fpitch + (int64_t)(out_off + o0 + o) * r + c]
                                          : 0.0f;
        }
    }

    // ---- staging and the K loop ---------------------------------------------------
    f32x16b acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
    // x B_m from the MFMA x operands: the two waves that share rows 64 wr ..
    // take one 32-row block each (block wc), so every SIMD does the same share;
    // lane (lc, hl) holds k 16 ks + 8 hl .. + 8 of row xbr
    const int32_t xbr = wr * 64 + 32 * wc + lc;
    const int32_t xbm = xbr < rows_here ? tr.member(P, xbr) : 0;  // its member in the tile
    float xb[RK];
#pragma unroll
    for (int c = 0; c < RK; ++c) xb[c] = 0.0f;

    if constexpr (DL) {
        // ---- direct-to-LDS pipeline ------------------------------------------------
        // As is in LDS before any stage load is issued: the barrier's fence
        // waits for its stores, with no stage load in flight yet
        __syncthreads();
        unsigned char* stg = smem;
        const int dr = lane >> 3, dc = (lane & 7) ^ (lane >> 3);  // row in the 8-row block, k chunk
        const uint16_t* xsrc[4];
        const uint16_t* wsrc[4];
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            // wave w fills blocks 4w .. 4w + 3 of x and of W; rows past the tile
            // read row 0 (finite values in rows and columns that are never stored)
            const int32_t R = 32 * wave + 8 * h + dr;
            xsrc[h] = static_cast<const uint16_t*>(P.x) +
                      tr.offset(P, R < rows_here ? R : 0, P.x_stride, P.x_plane) + dc * 8;
            wsrc[h] = Wb + (int64_t)(o0 + R < a ? o0 + R : 0) * kp + dc * 8;
        }
        // factor values: lane p holds member p / 16, floats (p % 16) * 4 .. of the
        // step's 64 k (every wave loads them: the same bytes)
        const bool f_on = noisy && lane < nm * 16;
        const float* fsrc = Fm + (f_on ? (int64_t)(lane >> 4) * fpitch + in_off + (lane & 15) * 4 : 0);
        auto issue = [&](int32_t st) {
            unsigned char* base = stg + (st & 1) * DL_SB;
#pragma unroll
            for (int h = 0; h < 4; ++h)
                __builtin_amdgcn_global_load_lds(xsrc[h] + st * DL_BK, base + (4 * wave + h) * 1024, 16, 0, 0);
#pragma unroll
            for (int h = 0; h < 4; ++h)
                __builtin_amdgcn_global_load_lds(wsrc[h] + st * DL_BK, base + DL_XB + (4 * wave + h) * 1024,
                                                 16, 0, 0);
            if (noisy && f_on)
                __builtin_amdgcn_global_load_lds(fsrc + (int64_t)st * DL_BK, base + DL_XB + DL_WB, 16, 0, 0);
        };
        const int32_t nkt = b / DL_BK;
        issue(0);
        // operand byte offsets (block and row); the chunk slot depends on the slice
        int32_t aoff[2], boff[4];
#pragma unroll
        for (int i = 0; i < 2; ++i) aoff[i] = (8 * wr + 4 * i + (lc >> 3)) * 1024 + (lc & 7) * 128;
#pragma unroll
        for (int j = 0; j < 4; ++j) boff[j] = DL_XB + (16 * wc + 4 * j + (lc >> 3)) * 1024 + (lc & 7) * 128;
        for (int32_t kt = 0; kt < nkt; ++kt) {
            vm_wait<0>();  // this wave's loads of stage kt (the only ones in flight)
            // every wave's loads of stage kt are in LDS, and every wave is done
            // with stage kt - 1, whose buffer the load of stage kt + 1 reuses
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);  // nothing of this step moves above the wait
            if (kt + 1 < nkt) issue(kt + 1);
            const unsigned char* base = stg + (kt & 1) * DL_SB;
            const float* Fs = reinterpret_cast<const float*>(base + DL_XB + DL_WB);
            // operand fragments one 16-wide k slice ahead: the reads of slice
            // ks + 1 are in flight while slice ks's MFMAs run
            auto frag = [&](int ks, u16x8 (&fa)[2], u16x8 (&fb)[4]) {
                const int32_t cx = ((2 * ks + hl) ^ (lc & 7)) << 4;  // this lane's k chunk slot
#pragma unroll
                for (int i = 0; i < 2; ++i) fa[i] = *reinterpret_cast<const u16x8*>(base + aoff[i] + cx);
#pragma unroll
                for (int j = 0; j < 4; ++j) fb[j] = *reinterpret_cast<const u16x8*>(base + boff[j] + cx);
            };
            // the factor values of k 16 ks + 8 hl .. + 8 of row xbr (the read
            // waits for the fragments already issued too)
            auto fvals = [&](int ks, float4 (&fv)[2]) {
                lds_f8_dl(Fs + xbm * DL_BK + 16 * ks + 8 * hl, fv[0], fv[1]);
            };
            auto slice = [&](const u16x8 (&fa)[2], const u16x8 (&fb)[4], const float4 (&fv)[2]) {
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[i][j] = mfma32b(fb[j], fa[i], acc[i][j]);
                if (noisy) {
                    // pairs of consecutive k: the factor rounded to bf16 as the
                    // register pipeline stages it
                    const uint4 x0 = __builtin_bit_cast(uint4, fa[0]), x1 = __builtin_bit_cast(uint4, fa[1]);
                    xb[0] = dot2_bf16(wc ? x1.x : x0.x, pack_bf16x2(fv[0].x, fv[0].y), xb[0]);
                    xb[0] = dot2_bf16(wc ? x1.y : x0.y, pack_bf16x2(fv[0].z, fv[0].w), xb[0]);
                    xb[0] = dot2_bf16(wc ? x1.z : x0.z, pack_bf16x2(fv[1].x, fv[1].y), xb[0]);
                    xb[0] = dot2_bf16(wc ? x1.w : x0.w, pack_bf16x2(fv[1].z, fv[1].w), xb[0]);
                }
            };
            static_assert(DL_BK == 64 && RK == 1, "four 16-wide k slices per stage, rank 1");
            u16x8 a0[2], b0[4], a1[2], b1[4];
            float4 f0[2], f1[2];
            frag(0, a0, b0);
            if (noisy) fvals(0, f0);
            frag(1, a1, b1);
            slice(a0, b0, f0);
            if (noisy) fvals(1, f1);
            frag(2, a0, b0);
            slice(a1, b1, f1);
            if (noisy) fvals(2, f0);
            frag(3, a1, b1);
            slice(a0, b0, f0);
            if (noisy) fvals(3, f1);
            slice(a1, b1, f1);
        }
        // the epilogue reuses stage 0 for x B_m: every wave is past its last read
        __syncthreads();
    } else {
        // ---- staging: thread -> x row tid / 2 and W row tid / 2, 32 k each ----------
        const int xr = tid >> 1, xk = (tid & 1) * 32;
        const bool xvalid = xr < rows_here;
        const int64_t xoff = xvalid ? tr.offset(P, xr, P.x_stride, P.x_plane) : 0;
        const int32_t wrow = o0 + xr;
        const bool wvalid = wrow < a;
        const uint16_t* wsrc = Wb + (int64_t)(wvalid ? wrow : 0) * kp + xk;
        constexpr int XU = XFMT == HSES_FMT_F32 ? 8 : 4;  // 16-byte loads of x per thread and step
        constexpr int XE = XFMT == HSES_FMT_F32 ? 4 : 8;  // elements per 16-byte load
        uint4 xv[XU], wv[4];
        uint32_t bv[KB_BPT];
        // staged factor words of this thread: (member, k pair, rank column), the
        // source of the pair's first k at step 0 (a step adds 64 rows)
        const float* bsrc[KB_BPT];
        int32_t bk2[KB_BPT];
        bool bon[KB_BPT];
    #pragma unroll
        for (int j = 0; j < KB_BPT; ++j) {
            const int32_t e = tid + KB_THREADS * j;  // [lm][kp][c]
            const int32_t c = e % RK, kp2 = (e / RK) % (KB_BK / 2), lm = e / (RK * (KB_BK / 2));
            bon[j] = noisy && e < bch && lm < nm && c < r;
            bk2[j] = 2 * kp2;
            bsrc[j] = Fm + (bon[j] ? lm * fpitch + (int64_t)(in_off + 2 * kp2) * r + c : 0);
        }
        auto load_step = [&](int32_t kt) {
            const int32_t k0 = kt * KB_BK + xk;
            // whole steps load unconditionally; the last, partial one masks
            if (xvalid && k0 + 32 <= b) {
    #pragma unroll
                for (int q = 0; q < XU; ++q) {
                    if constexpr (XFMT == HSES_FMT_F32)
                        xv[q] = reinterpret_cast<const uint4*>(static_cast<const float*>(P.x) + xoff + k0)[q];
                    else
                        xv[q] = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(P.x) + xoff + k0)[q];
                }
            } else {
    #pragma unroll
                for (int q = 0; q < XU; ++q) {
                    const bool ok = xvalid && k0 + XE * q < b;
                    if constexpr (XFMT == HSES_FMT_F32)
                        xv[q] = ok ? reinterpret_cast<const uint4*>(static_cast<const float*>(P.x) + xoff + k0)[q]
                                   : uint4{0, 0, 0, 0};
                    else
                        xv[q] = ok ? reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(P.x) + xoff + k0)[q]
                                   : uint4{0, 0, 0, 0};
                }
            }
            if (wvalid) {
    #pragma unroll
                for (int q = 0; q < 4; ++q) wv[q] = reinterpret_cast<const uint4*>(wsrc + kt * KB_BK)[q];
            } else {
    #pragma unroll
                for (int q = 0; q < 4; ++q) wv[q] = uint4{0, 0, 0, 0};
            }
            if (noisy) {
    #pragma unroll
                for (int j = 0; j < KB_BPT; ++j) {
                    const bool ok = bon[j] && kt * KB_BK + bk2[j] < b;  // b is even: both k of the pair
                    const float* p = bsrc[j] + (int64_t)kt * KB_BK * r;
                    bv[j] = ok ? pack_bf16x2(p[0], p[r]) : 0u;
                }
            }
        };
        auto store_step = [&](int buf) {
            uint16_t* xd = Xs + buf * KB_BUF + xr * KB_P + xk;
            if constexpr (XFMT == HSES_FMT_F32) {
    #pragma unroll
                for (int q = 0; q < XU; q += 2) {
                    const uint4 lo = xv[q], hi = xv[q + 1];
                    *reinterpret_cast<uint4*>(xd + 4 * q) = uint4{
                        pack_bf16x2(__uint_as_float(lo.x), __uint_as_float(lo.y)),
                        pack_bf16x2(__uint_as_float(lo.z), __uint_as_float(lo.w)),
                        pack_bf16x2(__uint_as_float(hi.x), __uint_as_float(hi.y)),
                        pack_bf16x2(__uint_as_float(hi.z), __uint_as_float(hi.w))};
                }
            } else {
    #pragma unroll
                for (int q = 0; q < XU; ++q) *reinterpret_cast<uint4*>(xd + 8 * q) = xv[q];
            }
            uint16_t* wd = Ws + buf * KB_BUF + xr * KB_P + xk;
    #pragma unroll
            for (int q = 0; q < 4; ++q) *reinterpret_cast<uint4*>(wd + 8 * q) = wv[q];
            if (noisy) {
    #pragma unroll
                for (int j = 0; j < KB_BPT; ++j) {
                    const int32_t e = tid + KB_THREADS * j;
                    if (e < bch) Bc[buf * bch + e] = bv[j];
                }
            }
        };

        const int32_t nkt = (b + KB_BK - 1) / KB_BK;
        load_step(0);
        store_step(0);
        __syncthreads();
        for (int32_t kt = 0; kt < nkt; ++kt) {
            const int cur = kt & 1;
            if (kt + 1 < nkt) load_step(kt + 1);
            const uint16_t* X = Xs + cur * KB_BUF;
            const uint16_t* W = Ws + cur * KB_BUF;
    #pragma unroll
            for (int ks = 0; ks < KB_BK / 16; ++ks) {
                const int kk = ks * 16 + hl * 8;
                u16x8 af[2], bf[4];
    #pragma unroll
                for (int i = 0; i < 2; ++i) af[i] = lds_u16x8(X + (wr * 64 + 32 * i + lc) * KB_P + kk);
    #pragma unroll
                for (int j = 0; j < 4; ++j) bf[j] = lds_u16x8(W + (wc * 128 + 32 * j + lc) * KB_P + kk);
                // D = W x^T: a lane's accumulator holds one output row (its x row)
                // and runs of four consecutive output columns
    #pragma unroll
                for (int i = 0; i < 2; ++i)
    #pragma unroll
                    for (int j = 0; j < 4; ++j) acc[i][j] = mfma32b(bf[j], af[i], acc[i][j]);
                if (noisy) {
                    // the factor's bf16 pairs of these 8 k: [lm][pair][c]
                    const uint4* bs = reinterpret_cast<const uint4*>(
                        Bc + cur * bch + (xbm * (KB_BK / 2) + ks * 8 + hl * 4) * RK);
                    const uint4 xw = __builtin_bit_cast(uint4, wc ? af[1] : af[0]);
                    const uint32_t xp[4] = {xw.x, xw.y, xw.z, xw.w};
                    if constexpr (RK == 1) {
                        const uint4 q = bs[0];  // pairs u = 0..3
                        xb[0] = dot2_bf16(xp[0], q.x, xb[0]);
                        xb[0] = dot2_bf16(xp[1], q.y, xb[0]);
                        xb[0] = dot2_bf16(xp[2], q.z, xb[0]);
                        xb[0] = dot2_bf16(xp[3], q.w, xb[0]);
                    } else {
    #pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            const uint4 q = bs[u];  // rank columns 0..3 of pair u
                            xb[0] = dot2_bf16(xp[u], q.x, xb[0]);
                            xb[1] = dot2_bf16(xp[u], q.y, xb[1]);
                            xb[2] = dot2_bf16(xp[u], q.z, xb[2]);
                            xb[3] = dot2_bf16(xp[u], q.w, xb[3]);
                        }
                    }
                }
            }
            if (kt + 1 < nkt) store_step(cur ^ 1);
            __syncthreads();
        }

    }

    // ---- epilogue: y = act(x W^T + (x B_m) A_m^T) ---------------------------------
    float* XBs = reinterpret_cast<float*>(Xs);  // [256][RK]; the buffers are free now
    if (noisy) {
#pragma unroll
        for (int c = 0; c < RK; ++c) {
            const float v = xb[c] + __shfl_xor(xb[c], 32);  // the two k groups
            if (hl == 0) XBs[xbr * RK + c] = v;
        }
        __syncthreads();
    }
    // One copy of the store loop per (activation, output format), chosen once.
    // With D = W x^T, accumulator element e of lane l is output row lc of the
    // 32-row block and column 8 (e / 4) + 4 hl + e % 4 of the 32-column tile:
    // each lane owns two rows and stores four consecutive columns at a time.
    const bool flat = P.n_time == 1;
    auto store_all = [&](auto actc, auto ybc) __attribute__((always_inline)) {
        constexpr int ACT = decltype(actc)::value;
        constexpr bool YB = decltype(ybc)::value;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int32_t row = wr * 64 + 32 * i + lc;
            if (row >= rows_here) continue;
            const int32_t lm = noisy ? tr.member(P, row) : 0;
            const int64_t yoff =
                (flat ? (L0 + row) * P.y_stride : tr.offset(P, row, P.y_stride, P.y_plane)) + o0;
            float xr_[RK];
#pragma unroll
            for (int c = 0; c < RK; ++c) xr_[c] = noisy ? XBs[row * RK + c] : 0.0f;
            if constexpr (YB) {
                if (vec_y == 2 && o0 + KB_BN <= a) {
                    // lanes l and l + 32 hold columns 8 g + 0..3 and 8 g + 4..7: after a
                    // swap of the upper half-lanes of group g with the lower of group
                    // g + 1, lane l holds the 8 columns of group g and lane l + 32 those
                    // of g + 1: one 16-byte store each
#pragma unroll
                    for (int j = 0; j < 4; ++j)
#pragma unroll
                        for (int g = 0; g < 4; g += 2) {
                            uint32_t w[2][2];
#pragma unroll
                            for (int h = 0; h < 2; ++h) {
                                const int32_t c0 = wc * 128 + 32 * j + 8 * (g + h) + 4 * hl;
                                float v[4];
#pragma unroll
                                for (int u = 0; u < 4; ++u) v[u] = acc[i][j][4 * (g + h) + u];
                                if (noisy) {
                                    const float* ar = As + ((size_t)lm * KB_BN + c0) * RK;
#pragma unroll
                                    for (int u = 0; u < 4; ++u) {
                                        float z = 0.0f;
#pragma unroll
                                        for (int c = 0; c < RK; ++c)
                                            z = __fadd_rn(z, __fmul_rn(xr_[c], ar[u * RK + c]));
                                        v[u] = __fadd_rn(v[u], z);
                                    }
                                }
#pragma unroll
                                for (int u = 0; u < 4; ++u) v[u] = act_value<ACT>(v[u]);
                                w[h][0] = pack_bf16x2(v[0], v[1]);
                                w[h][1] = pack_bf16x2(v[2], v[3]);
                            }
#pragma unroll
                            for (int q = 0; q < 2; ++q) {
                                const auto sw = __builtin_amdgcn_permlane32_swap(w[0][q], w[1][q], false, false);
                                w[0][q] = sw[0];
                                w[1][q] = sw[1];
                            }
                            const int32_t cs = wc * 128 + 32 * j + 8 * (g + hl);
                            *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(P.y) + yoff + cs) =
                                uint4{w[0][0], w[0][1], w[1][0], w[1][1]};
                        }
                    continue;
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int32_t col0 = wc * 128 + 32 * j + 8 * g + 4 * hl;
                    float v[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) v[u] = acc[i][j][4 * g + u];
                    if (noisy) {
                        const float* ar = As + ((size_t)lm * KB_BN + col0) * RK;
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            float z = 0.0f;
#pragma unroll
                            for (int c = 0; c < RK; ++c) z = __fadd_rn(z, __fmul_rn(xr_[c], ar[u * RK + c]));
                            v[u] = __fadd_rn(v[u], z);
                        }
                    }
#pragma unroll
                    for (int u = 0; u < 4; ++u) v[u] = act_value<ACT>(v[u]);
                    if (vec_y && o0 + col0 + 4 <= a) {
                        if constexpr (YB)
                            *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(P.y) + yoff + col0) =
                                uint2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
                        else
                            *reinterpret_cast<float4*>(P.y + yoff + col0) = float4{v[0], v[1], v[2], v[3]};
                    } else {
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            if (o0 + col0 + u >= a) continue;
                            if constexpr (YB)
                                reinterpret_cast<uint16_t*>(P.y)[yoff + col0 + u] = f2bf(v[u]);
                            else
                                P.y[yoff + col0 + u] = v[u];
                        }
                    }
                }
        }
    };
    using T0 = std::integral_constant<int, ACT_NONE>;
    using T1 = std::integral_constant<int, ACT_TANH>;
    using T2 = std::integral_constant<int, ACT_SIGMOID>;
    using T3 = std::integral_constant<int, ACT_RELU_SQ>;
    auto by_act = [&](auto ybc) __attribute__((always_inline)) {
        switch (act) {
            case ACT_TANH: store_all(T1{}, ybc); break;
            case ACT_SIGMOID: store_all(T2{}, ybc); break;
            case ACT_RELU_SQ: store_all(T3{}, ybc); break;
            default: store_all(T0{}, ybc); break;
        }
    };
    if (ybf16) by_act(std::true_type{});
    else by_act(std::false_type{});
}

static int32_t bf16_rk(int32_t r) { return r <= 1 ? 1 : 4; }

// Most members a 256-row tile (starting at a multiple of 256) can touch.
static int32_t bf16_nm_max(int32_t R, int32_t n) {
    int32_t nm;
    if (R % KB_BM == 0) nm = 1;
    else if (R > KB_BM) nm = 2;
    else if (KB_BM % R == 0) nm = KB_BM / R;
    else nm = (KB_BM - 1) / R + 2;
    return std::min(nm, n);
}

static int32_t bf16_kp(int32_t b) { return (b + KB_BK - 1) / KB_BK * KB_BK; }

struct Bf16Plan {
    int32_t rk, nm, bch, kp;
    bool dl;  // the direct-to-LDS pipeline
    size_t lds, w_bytes, f_bytes;
};

static bool bf16_plan(int32_t a, int32_t b, int32_t r, int32_t n, int32_t R, bool bf16_x, int32_t in_off,
                      Bf16Plan* pl) {
    if (a < KB_BN || b < 1 || n < 1 || r < 0 || r > KB_RMAX || b % 8) return false;
    pl->rk = bf16_rk(r);
    pl->nm = bf16_nm_max(R, n);
    pl->kp = bf16_kp(b);
    const size_t bch = r > 0 ? (size_t)pl->nm * (KB_BK / 2) * pl->rk : 0;
    if (bch > (size_t)KB_BPT * KB_THREADS) return false;
    pl->bch = (int32_t)bch;
    const size_t a_lds = r > 0 ? (size_t)pl->nm * KB_BN * pl->rk : 0;
    pl->lds = (size_t)4 * KB_BUF * 2 + (2 * bch + a_lds) * 4;
    // direct-to-LDS: bf16 x, whole 64-wide K steps, rank 0 or 1 (the factor
    // values of a step contiguous per member, 16-byte aligned, at most 1 KB)
    pl->dl = bf16_x && b % DL_BK == 0 && pl->rk == 1 &&
             (r == 0 || (pl->nm <= 4 && ((int64_t)(a + b) * r) % 4 == 0 && ((int64_t)in_off * r) % 4 == 0));
    if (pl->dl) pl->lds = (size_t)DL_NS * DL_SB + a_lds * 4;
    pl->w_bytes = align16((size_t)a * pl->kp * 2);
    pl->f_bytes = r > 0 ? align16((size_t)n * (a + b) * r * 4) : 0;
    return true;
}

size_t linear_bf16_workspace(int32_t a, int32_t b, int32_t r, int32_t n, int32_t rows_per_member,
                             int32_t n_time, int32_t math) {
    if (math != HSES_MATH_BF16 || (int64_t)rows_per_member * n_time > INT32_MAX) return 0;
    Bf16Plan pl;
    if (!bf16_plan(a, b, r, n, rows_per_member * n_time, false, 0, &pl)) return 0;
    return pl.w_bytes + pl.f_bytes;
}

int launch_linear_bf16(LinParams& P, DeviceState* st, hipStream_t s, void* work, size_t work_bytes,
                       int32_t act, int32_t y_fmt) {
    if (P.math != HSES_MATH_BF16) return HSES_ERR_UNSUPPORTED;
    if (P.x_fmt != HSES_FMT_F32 && P.x_fmt != HSES_FMT_BF16) return HSES_ERR_UNSUPPORTED;
    const int32_t r = (P.r > 0 && P.bs != 0.0f) ? P.r : 0;
    Bf16Plan pl;
    if (!bf16_plan(P.a, P.b, r, P.n, P.R, P.x_fmt == HSES_FMT_BF16, P.tmm ? P.a : 0, &pl) ||
        pl.lds > st->max_lds)
        return HSES_ERR_UNSUPPORTED;
    // 16-byte loads of 8 (bf16) or 4 (fp32) elements: aligned rows, whole groups
    const int64_t vec = P.x_fmt == HSES_FMT_F32 ? 4 : 8;
    if (reinterpret_cast<uintptr_t>(P.x) % 16 || P.x_stride % vec || (P.n_time > 1 && P.x_plane % vec))
        return HSES_ERR_UNSUPPORTED;
    if (!work || work_bytes < pl.w_bytes + pl.f_bytes) return HSES_ERR_UNSUPPORTED;
    const int64_t row_tiles = (P.total + KB_BM - 1) / KB_BM;
    const int64_t tiles = row_tiles * ((P.a + KB_BN - 1) / KB_BN);
    if (tiles > INT32_MAX) return set_error(HSES_ERR_INVALID_ARG, "too many output rows");
    uint16_t* Wb = static_cast<uint16_t*>(work);
    float* F = reinterpret_cast<float*>(static_cast<char*>(work) + pl.w_bytes);
    // four consecutive outputs per store (16 bytes fp32, 8 bytes bf16) when every
    // row start keeps them aligned (vec_y 1); bf16 rows 16-byte aligned: eight (2)
    const int64_t ybytes = y_fmt == HSES_FMT_BF16 ? 2 : 4;
    int32_t vec_y = reinterpret_cast<uintptr_t>(P.y) % (4 * ybytes) == 0 && P.y_stride % 4 == 0 &&
                    (P.n_time == 1 || P.y_plane % 4 == 0);
    if (vec_y && ybytes == 2 && reinterpret_cast<uintptr_t>(P.y) % 16 == 0 && P.y_stride % 8 == 0 &&
        (P.n_time == 1 || P.y_plane % 8 == 0))
        vec_y = 2;
    launch_w_to_bf16(P.W, P.a, P.b, pl.kp, P.tmm, Wb, s);
    HSES_CHECK_HIP(hipGetLastError());
    LinParams Q = P;
    Q.r = r;
    if (r > 0) {
        const int rc = launch_factors(Q, st, s, F);
        if (rc) return rc;
    }
    auto launch = [&](auto kern) -> int {
        HSES_CHECK_HIP(hipFuncSetAttribute((const void*)kern,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)pl.lds));
        hipLaunchKernelGGL(kern, dim3((uint32_t)tiles), dim3(KB_THREADS), pl.lds, s, Q,
                           (const uint16_t*)Wb, pl.kp, (const float*)F, pl.bch, act,
                           (int32_t)(y_fmt == HSES_FMT_BF16), vec_y);
        HSES_CHECK_HIP(hipGetLastError());
        return HSES_OK;
    };
    auto by_rk = [&](auto fmt) -> int {
        constexpr int X = decltype(fmt)::value;
        switch (pl.rk) {
            case 1: return launch(k_gemm_bf16<X, 1, false>);
            default: return launch(k_gemm_bf16<X, 4, false>);
        }
    };
    if (pl.dl) return launch(k_gemm_bf16<HSES_FMT_BF16, 1, true>);
    return P.x_fmt == HSES_FMT_F32 ? by_rk(std::integral_constant<int, HSES_FMT_F32>{})
                                   : by_rk(std::integral_constant<int, HSES_FMT_BF16>{});
}

}  // namespace hses
