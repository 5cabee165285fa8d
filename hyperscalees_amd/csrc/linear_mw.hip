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
//   k_mw_bits            the hidden-layer GEMM on those weights: each 256-row
//                        block's member's W tiles stream into LDS; waves of
//                        64 rows (every W fragment feeds two MFMAs); no B
//                        columns, no A block, no rank product; LIF fused.
#include "pair_bits.h"

namespace hses {

constexpr int MW_THREADS = 256;  // 4 waves: 32 rows of W each (a <= 128)
constexpr int MW_KC = 64;        // inputs (columns of W_m) per chunk
constexpr int MW_BP = K2_NMAX + 8;  // LDS pitch of a staged B row (fp16; 272 B)

// Elements of one member's weights: (a, kp) once (bf16) or twice (high then
// low part, fp16), each chunk-major: input chunk c (inputs 64 c .. + 63) of
// all a rows, [c][o][64], so that a 64-input chunk of a member is one
// contiguous run for its writer (k_member_weights) and its reader's tiles
// (k_mw_bits); chunk-strided rows spread writes over DRAM pages.
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

    // B staging: wave w stages rank rows 32w .. 32w + 31 of the chunk; its
    // load q covers rows 32w + 2 (lane / 4) + q % 2, inputs 16 (q / 2) +
    // 4 (lane % 4) .. + 3 (16 rows x 64 bytes per load, each 128-byte line
    // whole over two loads), so a thread holds the same 16 inputs of two
    // adjacent rank rows and stores their fp16 parts as pairs: 32-bit LDS
    // writes, lane l on bank 16 (l % 4) + l / 4 (conflict-free)
    const int32_t sc0 = 32 * wave + 2 * (lane >> 2), sk = 4 * (lane & 3);
    // 16-byte loads when every record row starts 16-byte aligned.  The record
    // and the member weights stream through once: non-temporal loads and
    // stores keep them from evicting W, which every pair re-reads from L2
    // (1.46 -> 1.29 ms at C3's fc1)
    const bool vec = ((uintptr_t)rec % 16 == 0) && (ab % 4 == 0);
    float4 bv[8];
    auto bload = [&](int32_t k0) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int32_t c = sc0 + (q & 1), k = k0 + 16 * (q >> 1) + sk;
            if (vec && c < r && k + 3 < b) {
                const f32x4 t = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(rp + (size_t)c * ab + k));
                bv[q] = make_float4(t[0], t[1], t[2], t[3]);
            } else {
                float e[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) e[u] = (c < r && k + u < b) ? rp[(size_t)c * ab + k + u] : 0.0f;
                bv[q] = make_float4(e[0], e[1], e[2], e[3]);
            }
        }
    };
    auto bstore = [&]() {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const float e0[4] = {bv[2 * kb].x, bv[2 * kb].y, bv[2 * kb].z, bv[2 * kb].w};
            const float e1[4] = {bv[2 * kb + 1].x, bv[2 * kb + 1].y, bv[2 * kb + 1].z,
                                 bv[2 * kb + 1].w};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                uint16_t h0, l0, h1, l1;
                split_f16(e0[u], &h0, &l0);
                split_f16(e1[u], &h1, &l1);
                const int32_t at = (16 * kb + sk + u) * MW_BP + sc0;  // even: 4-byte aligned
                *reinterpret_cast<uint32_t*>(Bh + at) = (uint32_t)h0 | ((uint32_t)h1 << 16);
                *reinterpret_cast<uint32_t*>(Bl + at) = (uint32_t)l0 | ((uint32_t)l1 << 16);
            }
        }
    };
    // W rows 16-byte aligned: 8 consecutive inputs as two float4
    const bool wvec = ((uintptr_t)W % 16 == 0) && (b % 4 == 0);
    const int32_t nch = kp / MW_KC;
    // this lane's runs of W for the chunk at k0 (run lane + 64 q: row
    // (lane + 64 q) / 8, inputs 8 (lane % 8) .. + 7), loaded before the
    // chunk's products so that the loads land while they run
    float wv[4][8];
    auto wload = [&](int32_t k0) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int32_t run = lane + 64 * q, o = o0 + (run >> 3), k = k0 + (run & 7) * 8;
            const float* wr = W + (size_t)min(o, a - 1) * b + k;
            if (wvec && k + 7 < b) {
                *reinterpret_cast<float4*>(wv[q]) = *reinterpret_cast<const float4*>(wr);
                *reinterpret_cast<float4*>(wv[q] + 4) = *reinterpret_cast<const float4*>(wr + 4);
            } else {
#pragma unroll
                for (int u = 0; u < 8; ++u) wv[q][u] = k + u < b ? wr[u] : 0.0f;
            }
        }
    };
    bload(0);
    bstore();
    __syncthreads();
    for (int32_t ch = 0; ch < nch; ++ch) {
        const int32_t k0 = ch * MW_KC;
        if (ch + 1 < nch) bload(k0 + MW_KC);
        if (wave_on) wload(k0);
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
                const int32_t o = o0 + row;
                if (o >= a) continue;
                float p[8];
                const float* w = wv[q];
                *reinterpret_cast<float4*>(p) = *reinterpret_cast<const float4*>(scr + row * MW_SP + k8);
                *reinterpret_cast<float4*>(p + 4) =
                    *reinterpret_cast<const float4*>(scr + row * MW_SP + k8 + 4);
                const int64_t at = (int64_t)ch * a * MW_KC + o * MW_KC + k8;
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
                        __builtin_nontemporal_store(eh, reinterpret_cast<u16x8*>(wm + off_even + at));
                        __builtin_nontemporal_store(el, reinterpret_cast<u16x8*>(wm + off_even + lo_off + at));
                    }
                    if (has_odd) {
                        __builtin_nontemporal_store(oh, reinterpret_cast<u16x8*>(wm + off_odd + at));
                        __builtin_nontemporal_store(ol, reinterpret_cast<u16x8*>(wm + off_odd + lo_off + at));
                    }
                } else {
                    u16x8 e, od;
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const float d = p[u] * (1.0f / K3_XSCALE);  // exact
                        e[u] = f2bf(w[u] + d);
                        od[u] = f2bf(w[u] - d);
                    }
                    if (has_even) __builtin_nontemporal_store(e, reinterpret_cast<u16x8*>(wm + off_even + at));
                    if (has_odd) __builtin_nontemporal_store(od, reinterpret_cast<u16x8*>(wm + off_odd + at));
                }
            }
        }
        // the next chunk's B after this chunk's stores: its loads had the
        // products and the stores' arithmetic to land
        if (ch + 1 < nch) bstore();
        __syncthreads();  // the next chunk's B is in LDS
    }
}

// ---- k_mw_bits: the forward on member weights -------------------------------
//
// y = x W_m^T for bit-packed x, the W_m of each 256-row block's member
// streamed from HBM (hses_member_weights' layout).  Four waves of 64 rows x
// all output columns: each W fragment read from LDS feeds the MFMAs of both
// of a wave's 32-row tiles, so a 32x32x16 MFMA needs half a fragment read
// (the factored kernel's waves of 32 rows need a whole one, which with one
// W fragment per MFMA saturates LDS bandwidth).  A wave's bit rows are staged
// by its own threads (thread t holds block row t), so they need no workgroup
// barrier.  W tiles (128 columns x 64 k, XOR-swizzled chunks as in
// k_pair_bits) stream by LDS DMA into NB buffers, each transfer issued right
// after the barrier that frees its buffer, NB - 1 tiles ahead (NB = 3 when a
// block has at least three stream tiles, so a transfer has two tiles of
// MFMAs to land; else 2); with X a stream tile holds 32 inputs of both
// parts, its k-steps alternating high and low part, so each expanded x
// operand feeds the MFMAs of two steps.  The epilogue runs the LIF (or
// stores y) in registers as k_pair_bits does, per row tile.  Two workgroups
// share a CU (58.6 KB of LDS each at b = 784).
constexpr int MB_THREADS = 256, MB_RB = 256;
constexpr int MB_XPF = 16;                  // x words per row (b <= 1024)
constexpr int MB_TILE = K2_NMAX * K2_BK;    // elements of one W tile buffer

struct MbLayout {
    size_t off_w, bytes;
    int32_t words;
    __host__ __device__ MbLayout(int b, int nb) {
        words = (b + 63) / 64;
        off_w = align16((size_t)MB_RB * words * 8);
        bytes = off_w + (size_t)nb * MB_TILE * 2;
    }
};

template <int EPI, int LT, bool SPK, bool RATE, bool X, int WT, int NB>
__global__ __launch_bounds__(MB_THREADS, 2) void k_mw_bits(const K2Args P) {
    static_assert(LT >= 1 && LT <= 16 && (LT & (LT - 1)) == 0, "T must be a power of two <= 16");
    static_assert(NB == 2 || NB == 3, "two or three tile buffers");
    extern __shared__ __align__(16) unsigned char smem[];
    const MbLayout lay(P.b, NB);
    uint64_t* Xbits = reinterpret_cast<uint64_t*>(smem);
    const uint32_t* Xbits32 = reinterpret_cast<const uint32_t*>(smem);
    uint16_t* WB = reinterpret_cast<uint16_t*>(smem + lay.off_w);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lc = lane & 31, hl = lane >> 5;
    const int32_t a = P.a, nkt = lay.words, kp = nkt * 64, R = P.R;
    // stream tiles per block; with X a tile is 32 inputs, and a last 64-input
    // chunk with 32 or fewer real inputs streams its first half only (C3's
    // fc1: 25 tiles for 784 inputs, not 26); at least two (the stream primes two)
    const int32_t ntb = X ? max(2, (P.b + 31) / 32) : nkt;
    const int32_t wrow0 = 64 * wave;
    // MFMA position p of a row tile -> its row: 8g + 4h + v -> 16h + 4g + v
    const int xrow = 16 * ((lc >> 2) & 1) + 4 * (lc >> 3) + (lc & 3);
    const int64_t part_off = X ? (int64_t)a * kp : 0;  // X: the low part after the high part

    // DMA: wave w's instruction q fills 1 KB chunk block 4w + q (staged columns
    // 32w + 8q .. + 7): lane l fetches chunk (l & 7) ^ ((column / 2) & 7) of
    // column 32w + 8q + l / 8; columns past a repeat row a - 1 (never stored)
    int32_t dl_off[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int32_t col = 32 * wave + 8 * q + (lane >> 3);
        const int32_t ch = (lane & 7) ^ (((8 * q + (lane >> 3)) >> 1) & 7);
        // X: chunk ch holds part (ch / 2) % 2 of inputs 16 (ch / 4) + 8 (ch % 2)
        // .. + 7 of the tile's 32, so k-steps 0-3 read high 0-15, low 0-15,
        // high 16-31, low 16-31
        dl_off[q] = min(col, a - 1) * K2_BK +
                    (X ? (int32_t)(((ch >> 1) & 1) * part_off) + 16 * (ch >> 2) + 8 * (ch & 1) : ch * 8);
    }
    // member weights are chunk-major (64-input chunks of a rows each), so a
    // tile is one contiguous 16 KB run (X: two 8 KB runs, one per part)
    auto dl_issue = [&](const uint16_t* src, int32_t t, int32_t buf) {
        if (wave >= WT) return;  // W rows no output tile reads
        const uint16_t* s = src + (X ? (size_t)(t >> 1) * a * K2_BK + (t & 1) * 32 : (size_t)t * a * K2_BK);
        const uint32_t dst = __builtin_amdgcn_readfirstlane(lds_addr(WB + buf * MB_TILE + (4 * wave) * 512));
#pragma unroll
        for (int q = 0; q < 4; ++q) lds_dma16(s + dl_off[q], dst + q * 1024);
    };
    // fragment of staged columns 32 ct + lc at k-step ks in buffer bsel
    const int32_t dl_u = hl ^ ((lc >> 1) & 7);
    auto frag_ptr = [&](int32_t bsel, int ks) -> const uint16_t* {
        return WB + bsel * MB_TILE + lc * K2_BK + (((2 * ks) ^ dl_u) << 3);
    };

    // work units: pair index and part (of P.split), as in k_pair_bits
    const int32_t G = (int32_t)gridDim.x, S = P.split;
    auto unit_of = [&](int32_t it, int32_t* pi_, int32_t* part) {
        if (S == 1) {
            *pi_ = (int32_t)blockIdx.x + it * G;
            *part = 0;
        } else {
            const int32_t xcd = (int32_t)blockIdx.x & 7, sl = (int32_t)blockIdx.x >> 3;
            *pi_ = it * (G / S) + xcd * (G / (8 * S)) + sl / S;
            *part = sl % S;
        }
    };
    auto unit_rows = [&](int32_t pi_, int32_t part, int64_t* lo, int64_t* hi) {
        const int32_t m_even = 2 * (P.pair_lo + pi_) - P.tid_lo;
        *lo = (int64_t)max(m_even, 0) * R;
        *hi = (int64_t)(min(m_even + 1, P.n - 1) + 1) * R;
        if (S > 1) {
            const int64_t span = (*hi - *lo) / S;  // a multiple of MB_RB (host check)
            *lo += part * span;
            *hi = *lo + span;
        }
    };
    auto unit_cursor = [&](int32_t pi_, int32_t part) {
        RowCursor c;
        c.m0 = max(2 * (P.pair_lo + pi_) - P.tid_lo, 0);
        c.q0 = 0;
        if (S > 1) {
            const int32_t off = part * (int32_t)((2 * (int64_t)R) / S);
            c.m0 += off / R;
            c.q0 = off - (off / R) * R;
        }
        return c;
    };
    auto advance = [&](RowCursor c) {
        c.q0 += MB_RB;
        if (c.q0 >= R) {
            const int32_t d = c.q0 / R;
            c.m0 += d;
            c.q0 -= d * R;
        }
        return c;
    };

    // bit rows: thread t holds row t of a block (its wave's rows only)
    uint64_t xv[MB_XPF];
    bool xv_ok = false;
    auto xload = [&](const RowCursor& cr, int64_t L, int64_t rhi) {
        const int32_t nv = (int32_t)min<int64_t>(rhi - L, MB_RB);
        xv_ok = tid < nv;
        int32_t m, q;
        cr.at(min(tid, nv - 1), R, &m, &q);
        const uint64_t* src = static_cast<const uint64_t*>(P.x) +
                              k2_phys(m, q, P.rpm, P.T, P.x_stride, P.x_plane);
#pragma unroll
        for (int w = 0; w < MB_XPF; ++w) xv[w] = src[min(w, nkt - 1)];
    };
    auto xstore = [&]() {
#pragma unroll
        for (int w = 0; w < MB_XPF; ++w) {
            if (w < nkt) Xbits[tid * nkt + w] = xv_ok ? xv[w] : 0ull;
            asm volatile("" ::"v"(xv[w]));  // every load consumed on every path
        }
    };

    int32_t dl_cb = 0;
    bool dl_primed = false, xready = false;
    // whether the last dl_issue_ahead issued (the tile that may stay in
    // flight at the next wait, NB = 3)
    bool iss_last = false;
    auto next_buf = [](int32_t c) { return c + 1 == NB ? 0 : c + 1; };
    // wait until the tile a barrier publishes has landed (NB = 3: the one
    // issued after it may stay in flight)
    auto dl_wait = [&]() {
        if (NB == 3 && iss_last)
            wait_vmcnt<4>();
        else
            wait_vmcnt<0>();
    };
    for (int32_t it = 0;; ++it) {
        int32_t pi, part;
        unit_of(it, &pi, &part);
        if (pi >= P.n_pairs) break;
        int64_t row_lo, row_hi;
        unit_rows(pi, part, &row_lo, &row_hi);
        int32_t pi_n, part_n;
        unit_of(it + 1, &pi_n, &part_n);
        const bool more_pairs = pi_n < P.n_pairs;
        RowCursor cur_rows = unit_cursor(pi, part);
        for (int64_t L0 = row_lo; L0 < row_hi; L0 += MB_RB) {
            const bool first = L0 == row_lo;
            const bool has_next = L0 + MB_RB < row_hi;
            const bool next_pair = !has_next && more_pairs;
            if (!first) cur_rows = advance(cur_rows);
            const int32_t nvalid = (int32_t)min<int64_t>(row_hi - L0, MB_RB);
            // this block's member's weights, and the next block's
            int32_t mn = cur_rows.m0;
            if (has_next)
                mn = cur_rows.q0 + MB_RB >= R ? cur_rows.m0 + 1 : cur_rows.m0;
            else if (more_pairs)
                mn = unit_cursor(pi_n, part_n).m0;
            const uint16_t* blk_src = P.wm + (size_t)cur_rows.m0 * P.wm_stride;
            const uint16_t* nblk_src = P.wm + (size_t)mn * P.wm_stride;
            if (first && !xready) {
                xload(cur_rows, L0, row_hi);
                xstore();
            }
            if (!dl_primed) {
                // the stream's first NB tiles (a block has at least NB)
                dl_issue(blk_src, 0, dl_cb);
                dl_issue(blk_src, 1, next_buf(dl_cb));
                if constexpr (NB == 3) {
                    dl_issue(blk_src, 2, next_buf(next_buf(dl_cb)));
                    wait_vmcnt<8>();
                } else {
                    wait_vmcnt<4>();
                }
                iss_last = true;
                dl_primed = true;
            }
            lds_barrier();

            // stream tile t (t >= ntb: the next block's tile t - ntb) into buf
            auto dl_issue_ahead = [&](int32_t t, int32_t buf) {
                iss_last = t < ntb || has_next || next_pair;
                if (t < ntb)
                    dl_issue(blk_src, t, buf);
                else if (iss_last)
                    dl_issue(nblk_src, t - ntb, buf);
            };

            f32x16 acc[2][WT];
            u16x8 fr[WT];
            {
                const uint16_t* tb = frag_ptr(dl_cb, 0);
#pragma unroll
                for (int ct = 0; ct < WT; ++ct) fr[ct] = lds_u16x8(tb + 32 * ct * K2_BK);
            }
            const uint32_t* xw[2] = {Xbits32 + (wrow0 + xrow) * (2 * nkt),
                                     Xbits32 + (wrow0 + 32 + xrow) * (2 * nkt)};
            uint32_t xw0[2] = {xw[0][0], xw[1][0]}, xw1[2] = {xw[0][1], xw[1][1]};
            // x operand of row tile rt at k-step ks from its tile word w
            auto expand = [&](uint32_t w, int ks) {
                const uint32_t xbyte = (w >> (8 * ((ks & 1) * 2 + hl))) & 0xffu;
                return X ? expand_bits_f16(xbyte) : expand_bits(xbyte);
            };
            // the x operands of the step about to run; each step expands the
            // next one's between its MFMAs (they do not depend on the MFMAs in
            // flight, so they issue while the matrix core is busy)
            u16x8 xa[2] = {expand(xw0[0], 0), expand(xw0[1], 0)};
            // one k-step: per column tile its two MFMAs and the read of its
            // fragment for the step at `nxt`; wn / ksn: the next step's words
            // and k-step
            // ksn < 0: the next step runs on the same x operands (X: the low
            // part's step after the high part's)
            auto step = [&](auto zc, const uint16_t* nxt, const uint32_t (&wn)[2], auto kc) {
                constexpr bool z = decltype(zc)::value;
                constexpr int ksn = decltype(kc)::value;
                u16x8 xn[2] = {xa[0], xa[1]};
#pragma unroll
                for (int ct = 0; ct < WT; ++ct) {
#pragma unroll
                    for (int rt = 0; rt < 2; ++rt) {
                        if constexpr (X)
                            acc[rt][ct] = mfma32_f16(xa[rt], fr[ct], z ? f32x16{} : acc[rt][ct]);
                        else
                            acc[rt][ct] = mfma32_bf16(xa[rt], fr[ct], z ? f32x16{} : acc[rt][ct]);
                    }
                    fr[ct] = lds_u16x8(nxt + 32 * ct * K2_BK);
                    if constexpr (ksn >= 0) {
                        if (ct == 0) xn[0] = expand(wn[0], ksn);
                        if (ct == (WT > 1 ? 1 : 0)) xn[1] = expand(wn[1], ksn);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                xa[0] = xn[0];
                xa[1] = xn[1];
            };
            using K0 = std::integral_constant<int, 0>;
            using K1 = std::integral_constant<int, 1>;
            using KS = std::integral_constant<int, -1>;
            auto tile = [&](int32_t kt, auto zc) {
                const bool more = kt + 1 < ntb;
                const int32_t kn = more ? kt + 1 : kt;
                const int32_t cb = dl_cb, nb = next_buf(dl_cb);
                const uint32_t wa[2] = {xw0[0], xw0[1]}, wb[2] = {xw1[0], xw1[1]};
                if constexpr (X) {
                    // 32 inputs (32-bit x word kt): high and low steps share
                    // the expanded x operands
                    step(zc, frag_ptr(cb, 1), wa, KS{});
                    step(std::false_type{}, frag_ptr(cb, 2), wa, K1{});
                    step(std::false_type{}, frag_ptr(cb, 3), wa, KS{});
                } else {
                    step(zc, frag_ptr(cb, 1), wa, K1{});
                    step(std::false_type{}, frag_ptr(cb, 2), wb, std::integral_constant<int, 2>{});
                    step(std::false_type{}, frag_ptr(cb, 3), wb, std::integral_constant<int, 3>{});
                }
                if (more) {
                    dl_wait();  // tile kt + 1 has landed
                    lds_barrier();
                    dl_issue_ahead(kt + NB, cb);
                }
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) {
                    if constexpr (X) {
                        xw0[rt] = xw[rt][kn];
                    } else {
                        xw0[rt] = xw[rt][2 * kn];
                        xw1[rt] = xw[rt][2 * kn + 1];
                    }
                }
                const uint32_t wn[2] = {xw0[0], xw0[1]};
                step(std::false_type{}, frag_ptr(more ? nb : cb, 0), wn, K0{});
                dl_cb = nb;
            };
            tile(0, std::true_type{});
            for (int32_t kt = 1; kt < ntb; ++kt) tile(kt, std::false_type{});
            // the next block's first tile has landed; its tile NB - 1 into the
            // last tile's buffer
            dl_wait();
            lds_barrier();
            dl_issue_ahead(ntb + NB - 1, NB == 3 ? next_buf(next_buf(dl_cb)) : next_buf(dl_cb));

            // the next block's bit rows land during the epilogue
            {
                int64_t nlo = L0, nhi = row_hi;
                RowCursor ncr = cur_rows;
                if (has_next) {
                    nlo = L0 + MB_RB;
                    ncr = advance(cur_rows);
                } else if (next_pair) {
                    unit_rows(pi_n, part_n, &nlo, &nhi);
                    ncr = unit_cursor(pi_n, part_n);
                }
                xload(ncr, nlo, nhi);
            }

            // acc[rt][jo][4g + v]: wave row 32 rt + 16 hl + 4g + v, column 32 jo + lc
            if constexpr (EPI == EPI_Y) {
#pragma unroll
                for (int rt = 0; rt < 2; ++rt)
#pragma unroll
                    for (int g = 0; g < 4; ++g)
#pragma unroll
                        for (int v = 0; v < 4; ++v) {
                            const int32_t row = wrow0 + 32 * rt + 16 * hl + 4 * g + v;
                            if (row >= nvalid) continue;
                            int32_t m, q;
                            cur_rows.at(row, R, &m, &q);
                            float* yrow = P.y + k2_phys(m, q, P.rpm, P.T, P.y_stride, P.y_plane);
#pragma unroll
                            for (int jo = 0; jo < WT; ++jo)
                                if (32 * jo + lc < a)
                                    yrow[32 * jo + lc] = X ? acc[rt][jo][4 * g + v] * (1.0f / K3_XSCALE)
                                                           : acc[rt][jo][4 * g + v];
                        }
            } else {
                // LIF (snn.rs:53-97) along each lane's rows, v = 0 at t = 0; the
                // reset as in k_pair_bits (charged kept when no spike, else 0)
                uint32_t wlo[2] = {0, 0}, whi[2] = {0, 0};  // lane u: spike words of wave row u
                // lanes of valid columns, as a ballot mask ANDed into each
                // step's ballot (a scalar AND instead of a per-lane select)
                uint64_t colmask[WT];
#pragma unroll
                for (int jo = 0; jo < WT; ++jo) colmask[jo] = __builtin_amdgcn_ballot_w64(32 * jo + lc < a);
                // X: the LIF runs on the 2^10-scaled currents the MFMAs leave
                // (membrane 2^10 v, threshold 2^10 v_th): scaling by a power of
                // two commutes with every rounding of the update, so the spikes
                // and resets are those of the unscaled recurrence
                const float vth = X ? P.v_th * K3_XSCALE : P.v_th;
                uint64_t dummy_carry;  // carry out of the count's add (unused)
                static_for<0, 2>([&](auto rc) {
                    constexpr int rt = decltype(rc)::value;
                    float vm[WT];
                    int32_t cnt[WT];
                    static_for<0, 16>([&](auto qc) {
                        constexpr int qq = decltype(qc)::value;  // 4g + v: time step qq % T
                        if constexpr (qq % LT == 0) {
#pragma unroll
                            for (int jo = 0; jo < WT; ++jo) {
                                vm[jo] = 0.0f;
                                cnt[jo] = 0;
                            }
                        }
                        uint64_t bal[WT];
#pragma unroll
                        for (int jo = 0; jo < WT; ++jo) {
                            const float c = acc[rt][jo][qq];
                            const float charged = __fadd_rn(vm[jo], __fmul_rn(__fadd_rn(-vm[jo], c), P.leak));
                            // one compare: its lane mask selects the reset and
                            // carries the count, and is the step's ballot
                            const uint64_t sp = __builtin_amdgcn_ballot_w64(charged >= vth);
                            float nv;
                            asm("v_cndmask_b32 %0, %1, 0, %2" : "=v"(nv) : "v"(charged), "s"(sp));
                            vm[jo] = nv;
                            if constexpr (RATE) {
                                int32_t nc;
                                asm("v_addc_co_u32 %0, %1, %2, 0, %3"
                                    : "=v"(nc), "=s"(dummy_carry)
                                    : "v"(cnt[jo]), "s"(sp));
                                cnt[jo] = nc;
                            }
                            if constexpr (SPK) bal[jo] = sp & colmask[jo];
                        }
                        if constexpr (RATE && qq % LT == LT - 1) {
                            const int32_t row = wrow0 + 32 * rt + 16 * hl + qq;
                            if (P.cpl) {
                                // the counts' bit planes (k_pair_bits' layout)
                                constexpr int NPL = LT == 1 ? 1 : LT == 2 ? 2 : LT == 4 ? 3 : LT == 8 ? 4 : 5;
                                uint64_t pb[NPL][WT];
#pragma unroll
                                for (int p = 0; p < NPL; ++p)
#pragma unroll
                                    for (int jo = 0; jo < WT; ++jo)
                                        pb[p][jo] = __builtin_amdgcn_ballot_w64((cnt[jo] >> p) & 1) & colmask[jo];
                                if (lc == 0 && row < nvalid) {
                                    int32_t m, q;
                                    cur_rows.at(row, R, &m, &q);
                                    uint64_t* dst = P.cpl + ((int64_t)m * P.rpm + q / LT) * P.cpl_stride;
                                    const int32_t words = (a + 63) >> 6;
#pragma unroll
                                    for (int p = 0; p < NPL; ++p)
#pragma unroll
                                        for (int hh = 0; hh < 2; ++hh) {
                                            const uint64_t b0 = 2 * hh < WT ? pb[p][min(2 * hh, WT - 1)] : 0ull;
                                            const uint64_t b1 = 2 * hh + 1 < WT ? pb[p][min(2 * hh + 1, WT - 1)] : 0ull;
                                            const uint64_t w = hl ? (b0 >> 32) | (b1 & 0xffffffff00000000ull)
                                                                  : (b0 & 0xffffffffull) | (b1 << 32);
                                            if (hh < words) dst[p * words + hh] = w;
                                        }
                                }
                            } else if (row < nvalid) {
                                int32_t m, q;
                                cur_rows.at(row, R, &m, &q);
                                float* rp = P.rate + ((int64_t)m * P.rpm + q / LT) * P.rate_stride;
#pragma unroll
                                for (int jo = 0; jo < WT; ++jo)
                                    if (32 * jo + lc < a) rp[32 * jo + lc] = (float)cnt[jo] * (1.0f / LT);
                            }
                        }
                        if constexpr (SPK) {
                            // ballot bit l: column 32 jo + l % 32 of wave row
                            // 32 rt + 16 (l / 32) + qq; lane 32 rt + 16 h + qq holds it
#pragma unroll
                            for (int hh = 0; hh < 2; ++hh) {
                                const uint64_t b0 = 2 * hh < WT ? bal[min(2 * hh, WT - 1)] : 0ull;
                                const uint64_t b1 = 2 * hh + 1 < WT ? bal[min(2 * hh + 1, WT - 1)] : 0ull;
                                put_lane<32 * rt + qq>(wlo[hh], whi[hh], (b0 & 0xffffffffull) | (b1 << 32));
                                put_lane<32 * rt + 16 + qq>(wlo[hh], whi[hh],
                                                            (b0 >> 32) | (b1 & 0xffffffff00000000ull));
                            }
                        }
                    });
                });
                if constexpr (SPK) {
                    const int32_t row = wrow0 + lane;
                    if (row < nvalid) {
                        int32_t m, q;
                        cur_rows.at(row, R, &m, &q);
                        uint64_t* dst = P.spk + k2_phys(m, q, P.rpm, LT, P.spk_stride, P.spk_plane);
                        dst[0] = ((uint64_t)whi[0] << 32) | wlo[0];
                        if (a > 64) dst[1] = ((uint64_t)whi[1] << 32) | wlo[1];
                    }
                }
            }
            // the next block's bit rows (this wave's own rows: a wave-level
            // order suffices; the next block's start barrier covers it too)
            xstore();
            xready = next_pair;
        }
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

// The forward on member weights: k_mw_bits over members
// [tid_lo, tid_lo + n), bit-packed x, rows per member a multiple of K3_RB.
int launch_linear_mw(LinParams& P, DeviceState* st, hipStream_t s, const LifOut* lif) {
    const bool xm = P.math == HSES_MATH_F32X;
    if (P.x_fmt != HSES_FMT_BITS || P.a > K2_NMAX || P.R % MB_RB || P.b > 64 * MB_XPF || P.tmm)
        return HSES_ERR_UNSUPPORTED;
    // the two-buffer stream needs two stream tiles per block: K of more than
    // one tile, or the split form (two stream tiles per 64 inputs)
    if (!xm && P.b <= 64) return HSES_ERR_UNSUPPORTED;
    if (lif && (P.n_time > 16 || (P.n_time & (P.n_time - 1)) != 0)) return HSES_ERR_UNSUPPORTED;
    // three tile buffers when a block streams at least three tiles
    const int32_t ntb = xm ? std::max(2, (P.b + 31) / 32) : (P.b + 63) / 64;  // as k_mw_bits counts them
    const int nbuf = ntb >= 3 ? 3 : 2;
    const MbLayout lay(P.b, nbuf);
    if (lay.bytes > st->max_lds) return HSES_ERR_UNSUPPORTED;
    K2Args A{};
    pair_range(P.tid_lo, P.n, &A.pair_lo, &A.n_pairs);
    // two workgroups per CU, persistent over the pairs
    const int32_t slots = 2 * st->num_cus;
    int32_t grid = std::max(1, std::min(A.n_pairs, slots));
    // pairs split over S workgroups of one XCD that work on them at the same
    // time: one 256-row block each when the pair's rows allow (S = 8 at C3),
    // so every block of a member streams the member's weights together and
    // they are fetched from HBM about once and re-read from that XCD's L2;
    // else 4, as in launch_linear_pair
    A.split = 1;
    for (int32_t S : {8, 4}) {
        if (P.tid_lo % 2 == 0 && P.n % 2 == 0 && (2 * (int64_t)P.R) % (S * MB_RB) == 0 &&
            slots % (8 * S) == 0 && (int64_t)A.n_pairs * S >= slots) {
            A.split = S;
            grid = slots;
            break;
        }
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
        hipLaunchKernelGGL(kern, dim3(grid), dim3(MB_THREADS), lay.bytes, s, A);
        HSES_CHECK_HIP(hipGetLastError());
        return HSES_OK;
    };
    auto by_math = [&](auto xc, auto nc) -> int {
        constexpr bool XX = decltype(xc)::value;
        constexpr int NB = decltype(nc)::value;
        if (!lif) {
            if (P.a <= 32) return launch(k_mw_bits<EPI_Y, 1, false, false, XX, 1, NB>);
            return launch(k_mw_bits<EPI_Y, 1, false, false, XX, 4, NB>);
        }
        const bool spk = lif->spk != nullptr, rate = lif->rate != nullptr || lif->cpl != nullptr;
        auto by_t = [&](auto sc, auto rc) -> int {
            constexpr bool S = decltype(sc)::value, Q = decltype(rc)::value;
            switch (P.n_time) {
                case 1: return launch(k_mw_bits<EPI_LIF, 1, S, Q, XX, 4, NB>);
                case 2: return launch(k_mw_bits<EPI_LIF, 2, S, Q, XX, 4, NB>);
                case 4: return launch(k_mw_bits<EPI_LIF, 4, S, Q, XX, 4, NB>);
                case 8: return launch(k_mw_bits<EPI_LIF, 8, S, Q, XX, 4, NB>);
                default: return launch(k_mw_bits<EPI_LIF, 16, S, Q, XX, 4, NB>);
            }
        };
        if (spk && rate) return by_t(std::true_type{}, std::true_type{});
        if (spk) return by_t(std::true_type{}, std::false_type{});
        return by_t(std::false_type{}, std::true_type{});
    };
    using nb2 = std::integral_constant<int, 2>;
    using nb3 = std::integral_constant<int, 3>;
    if (xm) return nbuf == 3 ? by_math(std::true_type{}, nb3{}) : by_math(std::true_type{}, nb2{});
    return nbuf == 3 ? by_math(std::false_type{}, nb3{}) : by_math(std::false_type{}, nb2{});
}

// ---- k_readout_counts: the readout on count planes, member weights in LDS ----
//
// The SNN readout (snn.rs:274-280: logits = rate W^T through do_mm,
// eggroll.rs:419-446) for a layer with few outputs and rows per member: one
// workgroup per pair stages the pair's A rows (r x a) in LDS, streams its B
// values from the factor record (coalesced over the inputs), forms
//   W_m[k][n] = W[k][n] + sign_m sum_c A'[k][c] B[n][c],  A' = A (sigma/sqrt(r))
// for both members (fp32 sums over c, one thread per (k, n) set), and then
// for every sample row of the two members decodes its spike counts from the
// P count planes (count = sum_p 2^p bit_p) and forms
//   y[k] = (sum_n count[n] W_m[k][n]) / T,
// the rate readout reassociated (the counts are exact, the 1/T a power of
// two).  Thread t of the logits phase takes sample t / 2 of the pair and the
// outputs k = t % 2, t % 2 + 2, ...
constexpr int RO_THREADS = 256, RO_KMAX = 32, RO_BMAX = 128;
// KQ: outputs in runs of 4 (a <= 4 KQ), so every output loop is unrolled
template <int KQ>
__global__ __launch_bounds__(RO_THREADS) void k_readout_counts(
    const uint64_t* __restrict__ cpl, int64_t cstride, int32_t T, int32_t P,
    const float* __restrict__ W, int32_t a, int32_t b, int32_t r, float bs, int32_t tid_lo,
    int32_t n, int32_t pair_lo, int32_t rpm, const float* __restrict__ rec,
    float* __restrict__ y, int64_t ystride) {
    extern __shared__ __align__(16) float ro_lds[];
    const int32_t pi = blockIdx.x, tid = threadIdx.x;
    const int32_t ab = a + b;
    const float* rp = rec + (size_t)pi * r * ab;
    const int32_t m_even = 2 * (pair_lo + pi) - tid_lo;  // -1: absent
    // the count planes of this thread's first task (phase 3), loaded first so
    // that they arrive during phases 1 and 2
    const int32_t words = (b + 63) >> 6;
    uint32_t plo0[5], phi0[5];
    auto load_planes = [&](int32_t task, uint32_t (&plo)[5], uint32_t (&phi)[5]) {
        const int32_t srow = task >> 1, wsel = task & 1;
        const int32_t half = srow / rpm, sl = srow - half * rpm;
        const int32_t m = m_even + half;
        const bool ok = task < 4 * rpm && m >= 0 && m < n && wsel < words;
        const uint64_t* pl = cpl + ((int64_t)(ok ? m : 0) * rpm + (ok ? sl : 0)) * cstride;
#pragma unroll
        for (int p = 0; p < 5; ++p) {
            const uint64_t v = (ok && p < P) ? pl[p * words + wsel] : 0ull;
            plo[p] = (uint32_t)v;
            phi[p] = (uint32_t)(v >> 32);
        }
    };
    load_planes(tid, plo0, phi0);
    // 1. the pair's A rows -> LDS as As[c][KP] (zero past a)
    constexpr int KP = 4 * KQ;
    float* As = ro_lds;
    for (int32_t idx = tid; idx < r * KP; idx += RO_THREADS) {
        const int32_t c = idx / KP, k = idx - c * KP;
        As[idx] = k < a ? rp[(size_t)c * ab + b + k] : 0.0f;
    }
    __syncthreads();
    // 2. d[k][n] = sum_c A[k][c] B[n][c]: thread t takes input n = t % b, all
    // outputs k < KP, and the ranks c = t / b, t / b + G, ... (G = 256 / b
    // groups, summed through LDS afterwards); B values straight from the
    // record (coalesced over n), a batch of ranks' loads in flight at once
    const int32_t G = RO_THREADS / b;  // >= 2 (b <= 128)
    const int32_t nn = tid % b, cg = tid / b;
    float d[KP];
#pragma unroll
    for (int k = 0; k < KP; ++k) d[k] = 0.0f;
    if (cg < G) {
        constexpr int CB = 16;
        for (int32_t c0 = cg; c0 < r; c0 += CB * G) {
            float bv[CB];
#pragma unroll
            for (int q = 0; q < CB; ++q) {
                const int32_t c = c0 + q * G;
                bv[q] = c < r ? __builtin_nontemporal_load(rp + (size_t)c * ab + nn) : 0.0f;
            }
#pragma unroll
            for (int q = 0; q < CB; ++q) {
                const int32_t c = min(c0 + q * G, r - 1);  // past r: bv = 0
                const float* ar = As + c * KP;
#pragma unroll
                for (int k4 = 0; k4 < KP; k4 += 4) {
                    const float4 a4 = *reinterpret_cast<const float4*>(ar + k4);
                    d[k4] = __builtin_fmaf(a4.x, bv[q], d[k4]);
                    d[k4 + 1] = __builtin_fmaf(a4.y, bv[q], d[k4 + 1]);
                    d[k4 + 2] = __builtin_fmaf(a4.z, bv[q], d[k4 + 2]);
                    d[k4 + 3] = __builtin_fmaf(a4.w, bv[q], d[k4 + 3]);
                }
            }
        }
    }
    float* part = ro_lds + r * KP;  // [group][n][KP]
    if (cg < G) {
#pragma unroll
        for (int k = 0; k < KP; ++k) part[(cg * b + nn) * KP + k] = d[k];
    }
    __syncthreads();
    if (cg == 0) {
        for (int32_t g = 1; g < G; ++g)
#pragma unroll
            for (int k = 0; k < KP; ++k) d[k] += part[(g * b + nn) * KP + k];
    }
    __syncthreads();  // the partials are no longer read
    // both members' weights into LDS, transposed: Wm[(member b + n) KP + k],
    // (sigma/sqrt(r)) applied to the sum (the forward scales A; the product
    // is the same up to rounding)
    const int32_t kp4 = KP;
    float* Wm = ro_lds + r * KP;
    if (cg == 0) {
#pragma unroll
        for (int k = 0; k < KP; ++k) {
            if (k < a) {
                const float w = W[(size_t)k * b + nn], dd = d[k] * bs;
                Wm[nn * KP + k] = w + dd;
                Wm[(b + nn) * KP + k] = w - dd;
            }
        }
    }
    __syncthreads();
    // 3. logits of the pair's 2 rpm sample rows: thread t takes sample t / 2
    // and the inputs of its 64-bit word t % 2 (b <= 128: two words), all
    // outputs; the two halves are added across the lane pair
    const float inv_t = 1.0f / (float)T;  // a power of two: exact
    for (int32_t task = tid; task < 4 * rpm; task += RO_THREADS) {
        const int32_t srow = task >> 1, wsel = task & 1;
        const int32_t half = srow / rpm, sl = srow - half * rpm;
        const int32_t m = m_even + half;
        const bool live = m >= 0 && m < n;
        uint32_t plo[5], phi[5];
        if (task == tid) {
#pragma unroll
            for (int p = 0; p < 5; ++p) {
                plo[p] = plo0[p];
                phi[p] = phi0[p];
            }
        } else {
            load_planes(task, plo, phi);
        }
        float acc[4 * KQ];
#pragma unroll
        for (int k = 0; k < 4 * KQ; ++k) acc[k] = 0.0f;
        const int32_t n0 = 64 * wsel, nend = min(b, n0 + 64);
        const float* wbase = Wm + (size_t)(half * b) * kp4;
        auto one = [&](int32_t nb, uint32_t cnt) {
            const float cf = (float)cnt;
            const float* wr = wbase + nb * kp4;
#pragma unroll
            for (int k4 = 0; k4 < 4 * KQ; k4 += 4) {
                const float4 w4 = *reinterpret_cast<const float4*>(wr + k4);
                acc[k4] = __builtin_fmaf(cf, w4.x, acc[k4]);
                acc[k4 + 1] = __builtin_fmaf(cf, w4.y, acc[k4 + 1]);
                acc[k4 + 2] = __builtin_fmaf(cf, w4.z, acc[k4 + 2]);
                acc[k4 + 3] = __builtin_fmaf(cf, w4.w, acc[k4 + 3]);
            }
        };
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const uint32_t(&src)[5] = hh ? phi : plo;
            const int32_t nlo = n0 + 32 * hh, nhi = min(nend, nlo + 32);
#pragma unroll 4
            for (int32_t nb = nlo; nb < nhi; ++nb) {
                const uint32_t sh = (uint32_t)(nb - nlo);
                uint32_t cnt = 0;
#pragma unroll
                for (int p = 0; p < 5; ++p) cnt |= __builtin_amdgcn_ubfe(src[p], sh, 1) << p;
                one(nb, cnt);
            }
        }
        // the lane pair (tasks 2 s, 2 s + 1 are lanes l, l ^ 1) holds the two words
#pragma unroll
        for (int k = 0; k < 4 * KQ; ++k) acc[k] += __shfl_xor(acc[k], 1);
        if (live && wsel == 0) {
            float* yr = y + ((int64_t)m * rpm + sl) * ystride;
#pragma unroll
            for (int k = 0; k < 4 * KQ; ++k)
                if (k < a) yr[k] = acc[k] * inv_t;
        }
    }
}

size_t readout_counts_lds(int32_t a, int32_t b, int32_t r) {
    // A rows [r][4 KQ], then the partials [G][b][4 KQ] (G b <= 256), which the
    // member weights [2][b][4 KQ] reuse
    const size_t kp4 = (size_t)((a + 3) & ~3);
    return ((size_t)r + RO_THREADS) * kp4 * 4;
}

int launch_readout_counts(const uint64_t* cpl, int64_t cstride, int32_t T, const float* W,
                          int32_t a, int32_t b, int32_t r, float bs, int32_t tid_lo, int32_t n,
                          int32_t rpm, const float* rec, float* y, int64_t ystride,
                          hipStream_t s) {
    if (a > RO_KMAX || b > RO_BMAX || 2 * rpm > RO_THREADS) return HSES_ERR_UNSUPPORTED;
    const size_t lds = readout_counts_lds(a, b, r);
    if (lds > 160 * 1024) return HSES_ERR_UNSUPPORTED;
    int32_t P = 1;
    while ((1 << (P - 1)) < T) ++P;
    if (P > 5) return HSES_ERR_UNSUPPORTED;
    int32_t lo, cnt;
    pair_range(tid_lo, n, &lo, &cnt);
    auto launch = [&](auto kern) -> int {
        if (lds > 64 * 1024)
            HSES_CHECK_HIP(hipFuncSetAttribute((const void*)kern,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        hipLaunchKernelGGL(kern, dim3((uint32_t)cnt), dim3(RO_THREADS), lds, s, cpl, cstride, T, P,
                           W, a, b, r, bs, tid_lo, n, lo, rpm, rec, y, ystride);
        HSES_CHECK_HIP(hipGetLastError());
        return HSES_OK;
    };
    switch ((a + 3) / 4) {
        case 1: return launch(k_readout_counts<1>);
        case 2: return launch(k_readout_counts<2>);
        case 3: return launch(k_readout_counts<3>);
        case 4: return launch(k_readout_counts<4>);
        case 5: return launch(k_readout_counts<5>);
        case 6: return launch(k_readout_counts<6>);
        case 7: return launch(k_readout_counts<7>);
        default: return launch(k_readout_counts<8>);
    }
}

}  // namespace hses
