// pair_bits.h -- the pair kernels' shared definitions and k_pair_bits.
//
// Included by linear_pair.hip (the factor draws, k_linear_pair, the pair
// forwards and their k_pair_bits instances) and linear_mw.hip (member
// weights and k_mw_bits, which reuses these definitions), which compile
// separately.  See linear_pair.hip for the design of the pair kernels.
#pragma once

#include <math.h>

#include <type_traits>

#include "linear_common.h"
#include "mfma.h"
#include "noise_dev.h"
#include "runtime.h"

namespace hses {

constexpr int K2_THREADS = 512, K2_RB = 256, K2_BK = 64, K2_NMAX = 128;
constexpr int K2_TP = K2_BK + 8;          // W/B tile pitch in bf16 elements (144 B)
constexpr int K2_COLS = 2 * K2_NMAX;      // staged columns per tile: W rows | B columns
constexpr int K2_LP = 20;                 // LIF transpose pitch (floats) per column
enum { EPI_Y = 0, EPI_LIF = 1 };

struct K2Layout {
    size_t off_a, off_xbits, off_wb, bytes;
    int32_t apitch, words, kp;
    __host__ __device__ K2Layout(int r, int b, bool bits) {
        // the second product steps K (= r) by 32: pad rows to a multiple of 32
        apitch = (r + 31) / 32 * 32 + 8;
        words = (b + 63) / 64;
        kp = words * 64;
        size_t o = align16(sizeof(BmTables));
        off_a = o;
        o = align16(o + (size_t)K2_NMAX * apitch * 2);
        off_xbits = o;
        if (bits) o = align16(o + (size_t)K2_RB * words * 8);
        off_wb = o;
        const size_t wb = (size_t)2 * K2_COLS * K2_TP * 2;  // two tile buffers
        const size_t xbs = (size_t)K2_RB * apitch * 2;      // epilogue alias
        bytes = o + (wb > xbs ? wb : xbs);
    }
};

// Rank column c of A is stored at column swap23(c) (bits 2 and 3 exchanged):
// the 8 rank columns one lane feeds to a 16-deep MFMA step of k_pair_bits,
// {0..3, 8..11} + 4 * k-group, then sit at 8 contiguous columns 8 * k-group.
__host__ __device__ __forceinline__ int32_t swap23(int32_t c) {
    return (c & ~12) | ((c & 4) << 1) | ((c & 8) >> 1);
}

// Operand image of one pair (factors drawn ahead, bf16): the input-side factor
// as [c][kp] (r rows, the layout of a staging slot, zero for k >= b), then
// the output-side factor as [o][swap23(c)] rows of K2_NMAX + 8 (a rows, zero
// for rank columns [r, r rounded up to 32)), the layout of k_pair_bits' LDS
// block.  Elements per pair: stride.
struct PairImage {
    size_t b_elems, stride;
    __host__ __device__ PairImage(int a, int b, int r) {
        b_elems = (size_t)r * ((b + 63) / 64 * 64);
        stride = b_elems + (size_t)a * (K2_NMAX + 8);
    }
};

// Split operand image of one pair (the fp32-accurate mode, HSES_MATH_F32X):
// each operand as a high and a low fp16 part, x = hi + lo to about 2^-22 of
// x (hi the fp16 rounding, lo the fp16 rounding of the remainder; x in
// {0, 1} is exact in fp16).  B_hi, B_lo as [c][kp] (zero for k >= b), then
// A_hi, A_lo as [o][swap23(c)] rows of K2_NMAX + 8 (zero for rank columns
// [r, r rounded up to 32)), A scaled by K3_XSCALE.  Elements per pair: stride.
struct PairImageX {
    size_t b_elems, a_elems, stride;
    __host__ __device__ PairImageX(int a, int b, int r) {
        b_elems = (size_t)r * ((b + 63) / 64 * 64);
        a_elems = (size_t)a * (K2_NMAX + 8);
        stride = 2 * b_elems + 2 * a_elems;
    }
};
// W and A enter the split products scaled by 2^10 (B and x B unscaled), so
// that A's low parts stay in fp16's normal range; the currents are the
// accumulators times 2^-10 (exact).
constexpr float K3_XSCALE = 1024.0f;

struct K2Args {
    const void* x;
    int64_t x_stride, x_plane;
    const uint16_t* wbf;  // W as bf16, (a, kp), zero for k >= b
    uint16_t* slots;      // per workgroup (r, kp) bf16 staging of B^T
    float* y;
    int64_t y_stride, y_plane;
    uint64_t key;
    const BmTables* tables;
    const uint32_t* log_exc;
    const uint32_t* cos_exc;
    const uint64_t* jump;
    uint64_t* spk;  // fused LIF: spike words (T, M, words), or NULL
    int64_t spk_stride, spk_plane;
    float* rate;    // fused LIF: spike counts / T (M, a), or NULL
    int64_t rate_stride;
    // fused LIF: spike-count bit planes in place of the rates, or NULL: output
    // row (m, s) has log2(T) + 1 planes of words(a) words at cpl + (m rpm + s)
    // cpl_stride, bit c of plane p being bit p of neuron c's count
    uint64_t* cpl;
    int64_t cpl_stride;
    int32_t a, b, r, R, rpm, T, n, tid_lo, pair_lo, n_pairs, epoch, nreuse;
    int32_t segs;   // generation segments per stream row (jump table for row length r / segs)
    int32_t group;  // pairs generated together (k_linear_pair; their A rows share the LDS block)
    int32_t tmm;    // do_Tmm stream roles (LinParams::tmm)
    int32_t x_vec;  // dense x: strides keep 8-element groups 16-byte aligned
    // bit-packed x in the packed time-inner layout (x_plane = a row's words,
    // x_stride = T rows of them): row L of the call lies at word L * words,
    // so a block's bit rows are one contiguous run, 16-byte aligned
    int32_t x_packed;
    // k_pair_bits work units: each pair's row blocks split evenly over `split`
    // workgroups (1, or 4 with every pair full and the grid a multiple of 32),
    // which work on it at the same time on one XCD (workgroups are dealt to
    // the 8 XCDs in turn), so the pair's operand image is fetched from HBM
    // about once and re-read from that XCD's L2
    int32_t split;
    float bs, leak, v_th;
    // Factor record (do_mm), or NULL: pair pair_lo + i's raw normals (before
    // any scale) at rec[(i * r + c) * (a + b) + j] for stream row j, rank c.
    float* rec;
    // Factors drawn ahead (PRE kernels, k_pair_gen): pair pair_lo + i's
    // operand image (PairImage) at bimg + i * stride.
    uint16_t* bimg;
    // Member weights (k_mw_bits): member tid_lo + m's perturbed W (the
    // member_weights layout, (a, kp) per part) at wm + m * wm_stride.
    const uint16_t* wm;
    int64_t wm_stride;
};

// bm_run that also stores each raw normal i at rp[i * pitch] when rp is set
// (the factor record; one branch per row, not per normal).
template <typename Sink>
__device__ __forceinline__ void bm_rec_run(uint64_t& s, int32_t count, const NoiseCtx& ctx,
                                           float* rp, int32_t pitch, Sink sink) {
    if (rp)
        bm_run(s, count, ctx, [&](int32_t i, float v) {
            rp[(size_t)i * pitch] = v;
            sink(i, v);
        });
    else
        bm_run(s, count, ctx, sink);
}

// Stream row j of a pair's factor stream: input-side operand row (staged in
// the slot as [c][k]) or output-side row (LDS, [o][c]), and its scale.
// do_mm: rows [0, b) input side, [b, a + b) output side scaled by sigma/sqrt(r);
// do_Tmm: rows [0, a) output side, [a, a + b) input side scaled.
struct StreamRow {
    bool in_side;
    int32_t row;
    float scale;
    __device__ __forceinline__ StreamRow(const K2Args& P, int32_t j) {
        const int32_t f0 = P.tmm ? P.a : 0;
        in_side = j >= f0 && j < f0 + P.b;
        row = in_side ? j - f0 : (P.tmm ? j : j - P.b);
        scale = (in_side == (P.tmm != 0)) ? P.bs : 1.0f;
    }
};

// Rows of a block are addressed relative to the block start L0 = m0 * R + q0:
// row L0 + i belongs to member m0 or m0 + 1 (a block never leaves its pair),
// so a conditional subtraction replaces 64-bit division.
struct RowCursor {
    int32_t m0, q0;
    __device__ __forceinline__ void at(int32_t i, int32_t R, int32_t* m, int32_t* q) const {
        int32_t qq = q0 + i, mm = m0;
        if (qq >= R) {
            qq -= R;
            ++mm;
        }
        *m = mm;
        *q = qq;
    }
};

// Physical element offset of row q (slot-major: q = s * T + t) of member m.
__device__ __forceinline__ int64_t k2_phys(int32_t m, int32_t q, int32_t rpm, int32_t T,
                                           int64_t stride, int64_t plane) {
    const int32_t s = (int32_t)((uint32_t)q / (uint32_t)T);
    const int32_t t = q - s * T;
    return t * plane + ((int64_t)m * rpm + s) * stride;
}

// fp32 -> fp16 high part and fp16 low part (round to nearest even both):
// hi + lo is v to about 2^-22 of v (v - hi is exact in fp32).
__device__ __forceinline__ void split_f16(float v, uint16_t* hi, uint16_t* lo) {
    const _Float16 h = (_Float16)v;
    *hi = __builtin_bit_cast(uint16_t, h);
    *lo = __builtin_bit_cast(uint16_t, (_Float16)(v - (float)h));
}

// Workgroup barrier that orders LDS accesses only: global loads issued
// before it stay in flight (a plain __syncthreads also waits for every
// outstanding global load, which would drain the tile prefetch).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Orders a wave's own LDS accesses (the writes before, the reads after).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// v_writelane_b32 through the compiler intrinsic, so the hazard recognizer
// inserts the wait states between the SGPR write (the ballot's compare) and
// its read by the lane write.
extern "C" __device__ int32_t hses_writelane_i32(int32_t src, int32_t lane, int32_t old)
    __asm("llvm.amdgcn.writelane.i32");

// Lane L of (lo, hi) <- the wave-uniform 64-bit value w (no lane masks).
template <int L>
__device__ __forceinline__ void put_lane(uint32_t& lo, uint32_t& hi, uint64_t w) {
    lo = (uint32_t)hses_writelane_i32((int32_t)(uint32_t)w, L, (int32_t)lo);
    hi = (uint32_t)hses_writelane_i32((int32_t)(uint32_t)(w >> 32), L, (int32_t)hi);
}

__device__ __forceinline__ uint4 mask4(uint4 v, uint32_t m) {
    return uint4{v.x & m, v.y & m, v.z & m, v.w & m};
}

// ---- k_pair_bits: bit-packed input, epilogue in registers ----------------------
//
// The hidden-layer form of the pair kernel (x bit-packed, bf16 MFMA 32x32x16).
// Eight waves of 32 rows x all 256 staged columns (128 W rows | 128 rank
// columns of B), so every wave owns whole output rows and the epilogue needs
// no LDS round trip:
//   * the B columns are accumulated transposed (mfma(B, x)): lane l then holds
//     16 rank columns of the row at MFMA position l % 32, which after the
//     member sign and the bf16 rounding are the A-operand fragments of the
//     second product (xB) A^T as they are (the k-group of each 16-step is
//     chosen to match, and A is read with the same mapping);
//   * a 32x32 accumulator gives lane l the 16 rows 8g + 4h + v (h = l / 32)
//     of column l % 32; block rows are assigned so that those are wave rows
//     16h + 4g + v, i.e. 16 consecutive rows.  With slot-major rows each
//     T-step series (T <= 16) of a column sits in one lane and the LIF runs
//     in registers; the comparison of a step, as a ballot, holds two rows x
//     32 columns, so its 32-bit halves are the halves of spike words.
// Each x bit row is expanded by one wave only.  The next block's bit rows and
// first W/B tile are loaded while the epilogue runs.
constexpr int K3_THREADS = 512, K3_RB = 256;
// Bit-row staging: thread t handles row t / 2 and words t % 2, t % 2 + 2, ...
// (at most K3_XPF of them: rows of up to 2 * K3_XPF words, b <= 1024; wider
// inputs use k_linear_pair).
constexpr int K3_XPF = 8;
// A pitch in bf16: r <= 128 padded to 128, plus 8, so rows start 16-byte
// aligned and the 16 rows of a quarter-wave's 16-byte reads (row stride 68
// dwords) cover distinct banks; a compile-time constant keeps the second
// product's LDS addresses immediate offsets of one base.
constexpr int K3_AP = K2_NMAX + 8;


typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16 mfma32_bf16(const u16x8& a, const u16x8& b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ f32x16 mfma32_f16(const u16x8& a, const u16x8& b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Two floats as packed fp16 high parts and packed fp16 low parts (split_f16
// on each).
__device__ __forceinline__ void split_f16x2(float v0, float v1, uint32_t* hi, uint32_t* lo) {
    uint16_t h0, l0, h1, l1;
    split_f16(v0, &h0, &l0);
    split_f16(v1, &h1, &l1);
    *hi = (uint32_t)h0 | ((uint32_t)h1 << 16);
    *lo = (uint32_t)l0 | ((uint32_t)l1 << 16);
}

// Direct-to-LDS tiles (DL): K3_DLBUF unpadded tile buffers of K2_COLS
// columns x K2_BK k (128 bytes per column), filled by LDS DMA (each lane's
// 16-byte chunk lands at the wave's base + 16 x lane).  A column's eight
// 16-byte chunks are stored XOR-swizzled, chunk c at slot c ^ ((column / 2) & 7),
// so that the 16 lanes of a fragment read (16 columns, one chunk each) cover
// all 64 banks.
constexpr int K3_DLBUF = 3;
constexpr int K3_DLTILE = K2_COLS * K2_BK;  // bf16 elements per DL tile buffer

struct K3Layout {
    size_t off_a, off_xbits, off_wb, bytes;
    int32_t apitch, words, kp;
    // dl: the DL form (factors drawn ahead, so no noise tables); x: the
    // split (fp32-accurate) form, A as high and low parts and two DL buffers
    __host__ __device__ K3Layout(int r, int b, bool dl = false, bool x = false) {
        apitch = K3_AP;
        words = (b + 63) / 64;
        kp = words * 64;
        size_t o = dl ? 0 : align16(sizeof(BmTables));
        off_a = o;
        o = align16(o + (size_t)(x ? 2 : 1) * K2_NMAX * apitch * 2);
        off_xbits = o;
        o = align16(o + (size_t)K3_RB * words * 8);
        off_wb = o;
        bytes = o + (dl ? (size_t)(x ? 2 : K3_DLBUF) * K3_DLTILE * 2
                        : (size_t)2 * K2_COLS * K2_TP * 2);
    }
};

// One LDS DMA of 16 bytes per lane: lane l's 16 bytes at gptr land at LDS byte
// address lds + 16 l (lds wave-uniform).  Written as inline assembly so that
// the compiler's memory model does not see an LDS write that completes on the
// vector-memory counter: its LDS fences would otherwise wait for every
// transfer in flight, including the tile streaming two ahead.  The kernel
// orders these transfers itself (wait_vmcnt before the barrier that
// publishes a tile).
__device__ __forceinline__ void lds_dma16(const void* gptr, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "s"(lds)
                 : "memory", "m0");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// s_waitcnt on the vector-memory counter only (gfx9 encoding: vmcnt in bits
// 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// EPI_Y: store the currents; EPI_LIF: LIF with T = LT, spike words if SPK,
// spike rates if RATE.  PRE: the factors were drawn ahead (k_pair_gen): A
// comes from the record, B from the operand image, and nothing is generated.
// DL (with PRE, K of more than two tiles): the W/B tiles stream into three
// LDS buffers by LDS DMA, two tiles ahead of the MFMAs, instead of through
// registers; the stream runs on across blocks and pairs.
// X (with DL): the split fp16 operands of the fp32-accurate mode (P.bimg a
// PairImageX image, P.wbf W's high then low part, scaled): each K tile is
// taken twice, its high and its low part (two DL buffers; each transfer is
// issued right after the barrier that frees its buffer, one tile ahead), and
// the second product is (xB)_hi A_hi + (xB)_lo A_hi + (xB)_hi A_lo.
// WT: output tiles of 32 columns computed (4; 1 for a <= 32, where the other
// three would only be discarded).
template <int EPI, int LT, bool SPK, bool RATE, bool PRE = false, bool DL = false, bool X = false,
          int WT = 4>
__global__ __launch_bounds__(K3_THREADS) void k_pair_bits(const K2Args P) {
    static_assert(LT >= 1 && LT <= 16 && (LT & (LT - 1)) == 0, "T must be a power of two <= 16");
    static_assert(!DL || PRE, "the DL tile stream needs factors drawn ahead");
    static_assert(!X || DL, "the split operands stream through DL buffers");
    // two DL buffers, each transfer issued right after the barrier that frees
    // its buffer (X); or three, two tiles ahead
    constexpr bool EARLY = X;
    constexpr int NBUF = EARLY ? 2 : K3_DLBUF;  // DL tile buffers
    constexpr int DIST = NBUF - 1;              // tiles the stream runs ahead
    extern __shared__ __align__(16) unsigned char smem[];
    const K3Layout lay(P.r, P.b, DL, X);
    BmTables* tabs = reinterpret_cast<BmTables*>(smem);
    uint16_t* As = reinterpret_cast<uint16_t*>(smem + lay.off_a);
    uint64_t* Xbits = reinterpret_cast<uint64_t*>(smem + lay.off_xbits);
    const uint32_t* Xbits32 = reinterpret_cast<const uint32_t*>(smem + lay.off_xbits);
    uint16_t* WB = reinterpret_cast<uint16_t*>(smem + lay.off_wb);  // [2][K2_COLS][K2_TP]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lc = lane & 31, hl = lane >> 5;  // MFMA column / k-group of this lane
    const int32_t r = P.r, a = P.a, b = P.b, kp = lay.kp, nkt = lay.words, R = P.R;
    const int32_t rp32 = (r + 31) & ~31;
    uint16_t* slot = PRE ? nullptr : P.slots + (size_t)blockIdx.x * r * kp;

    if constexpr (!PRE) {
        load_bm_tables(tabs, P.tables);
        for (int32_t i = tid; i < r * (kp - b); i += K3_THREADS) {
            const int32_t c = i / (kp - b), k = b + i % (kp - b);
            slot[(size_t)c * kp + k] = 0;
        }
        __threadfence_block();
        __syncthreads();
    }
    const NoiseCtx ctx{tabs, P.log_exc, P.cos_exc};

    // Tile loader: thread -> (staged column, 32-k half); columns [0, 128) are
    // W rows, [128, 256) rank columns of B; absent ones are staged as zeros.
    const int lcol = tid >> 1, lk = (tid & 1) * 32;
    const bool lvalid = lcol < K2_NMAX ? lcol < a : lcol - K2_NMAX < r;
    const size_t loff = (size_t)(lcol < K2_NMAX ? min(lcol, a - 1) : min(lcol - K2_NMAX, r - 1)) * kp + lk;
    const uint16_t* lsrc = (lcol < K2_NMAX ? P.wbf : slot) + loff;  // PRE: B part set per pair
    uint16_t* ldst = WB + lcol * K2_TP + lk;
    const uint32_t lmask = lvalid ? 0xffffffffu : 0u;
    // DL: wave w's DMA instruction q fills chunk block 4w + q of a tile buffer
    // (staged columns 32w + 8q .. 32w + 8q + 7); lane l fetches chunk
    // (l & 7) ^ swizzle of column 32w + 8q + l / 8.  Waves 0-3 stage W rows,
    // waves 4-7 rank columns of B; absent columns repeat the last present one
    // (their outputs are never stored, and A is zero there).
    int32_t dl_off[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int32_t col = 32 * wave + 8 * q + (lane >> 3);
        const int32_t ch = (lane & 7) ^ (((8 * q + (lane >> 3)) >> 1) & 7);
        const int32_t srow = col < K2_NMAX ? min(col, a - 1) : min(col - K2_NMAX, r - 1);
        dl_off[q] = srow * kp + ch * 8;
    }
    auto dl_issue = [&](const uint16_t* src, int32_t kt, int32_t buf) {
        if (wave >= WT && wave < 4) return;  // W rows no output tile reads
        const uint32_t dst = __builtin_amdgcn_readfirstlane(
            lds_addr(WB + buf * K3_DLTILE + (4 * wave) * 512));
#pragma unroll
        for (int q = 0; q < 4; ++q) lds_dma16(src + dl_off[q] + kt * K2_BK, dst + q * 1024);
    };
#define K3_TILE_LOAD(kt)                                                            \
    do {                                                                            \
        const uint4* src_ = reinterpret_cast<const uint4*>(lsrc + (kt) * K2_BK);    \
        pf0 = src_[0];                                                              \
        pf1 = src_[1];                                                              \
        pf2 = src_[2];                                                              \
        pf3 = src_[3];                                                              \
    } while (0)
#define K3_TILE_STORE(buf)                                                          \
    do {                                                                            \
        uint4* d_ = reinterpret_cast<uint4*>(ldst + (buf) * (K2_COLS * K2_TP));     \
        d_[0] = mask4(pf0, lmask);                                                  \
        d_[1] = mask4(pf1, lmask);                                                  \
        d_[2] = mask4(pf2, lmask);                                                  \
        d_[3] = mask4(pf3, lmask);                                                  \
    } while (0)
    // Wave row of MFMA position p (0..31): 8g + 4h + v -> 16h + 4g + v.
    const int xrow = 16 * ((lc >> 2) & 1) + 4 * (lc >> 3) + (lc & 3);
    const int32_t wrow0 = wave * 32;
    const int32_t xs_row = tid >> 1, xs_w = tid & 1;
    // Rows [lo, hi) of the members of pair index pi.
    auto pair_rows = [&](int32_t pi_, int64_t* lo, int64_t* hi) {
        const int32_t m_even = 2 * (P.pair_lo + pi_) - P.tid_lo;
        *lo = (int64_t)max(m_even, 0) * R;
        *hi = (int64_t)(min(m_even + 1, P.n - 1) + 1) * R;
    };
    bool xready = false;  // the first block's bit rows are already in LDS
    // K of at most two tiles: both stay in the two LDS buffers for all of a
    // pair's blocks (staged by its first block), so no block reloads them
    // and the K loop needs no barrier between its tiles.
    const bool resident = DL ? false : nkt <= 2;
    // DL tile stream: the buffer of the block's current tile, and whether the
    // stream has been started (tiles 0 and 1 of the first block).
    int32_t dl_cb = 0;
    bool dl_primed = false;
    const uint16_t* dl_wsrc = wave < 4 ? P.wbf : nullptr;  // waves 4-7: set per pair
    const size_t dl_stride = X ? PairImageX(a, b, r).stride : PairImage(a, b, r).stride;
    // X: a stream tile t is K tile t / 2, its high (t even) or low part
    const int32_t dl_part = wave < 4 ? a * kp : r * kp;
    const int32_t nt = X ? 2 * nkt : nkt;  // stream tiles per block
    auto dl_issue_t = [&](const uint16_t* src, int32_t t, int32_t buf) {
        if constexpr (X)
            dl_issue(src + (t & 1) * dl_part, t >> 1, buf);
        else
            dl_issue(src, t, buf);
    };

    // Work unit `it` of this workgroup: pair index and part (of P.split).
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
    // Rows [lo, hi) of part `part` of pair pi, and the (member, row) of lo.
    auto unit_rows = [&](int32_t pi_, int32_t part, int64_t* lo, int64_t* hi) {
        pair_rows(pi_, lo, hi);
        if (S > 1) {
            const int64_t span = (*hi - *lo) / S;  // a multiple of K3_RB (host check)
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

    for (int32_t it = 0;; ++it) {
        int32_t pi, part;
        unit_of(it, &pi, &part);
        if (pi >= P.n_pairs) break;
        const int32_t pair = P.pair_lo + pi;
        int64_t row_lo, row_hi;
        unit_rows(pi, part, &row_lo, &row_hi);
        int32_t pi_n, part_n;  // this workgroup's next unit
        unit_of(it + 1, &pi_n, &part_n);
        const bool more_pairs = pi_n < P.n_pairs;
        // DL: this wave's tile source for pair pi and for the next unit's pair
        const uint16_t* dl_src = wave < 4 ? dl_wsrc : P.bimg + (size_t)pi * dl_stride;
        const uint16_t* dl_src_next =
            wave < 4 ? dl_wsrc : P.bimg + (size_t)(more_pairs ? pi_n : pi) * dl_stride;

        // ---- 1. factors: A rows -> LDS (bf16, [o][c]); B rows -> slot ([c][k]) ----
        if constexpr (PRE) {
            // the pair's image holds A in this block's layout: one round of
            // 16-byte copies (a rows of K3_AP bf16, at most 5 per thread)
            const PairImage im(a, b, r);
            const PairImageX imx(a, b, r);
            const uint16_t* img = P.bimg + (size_t)pi * (X ? imx.stride : im.stride);
            if (lcol >= K2_NMAX) lsrc = img + loff;
            // X: A's high then low part (a rows each), as they lie in the image
            const uint4* asrc = reinterpret_cast<const uint4*>(img + (X ? 2 * imx.b_elems : im.b_elems));
            const int32_t n16 = (X ? 2 : 1) * a * (K3_AP / 8);
            uint4 av0, av1, av2, av3, av4;
            auto aload = [&](int q) { return asrc[min(tid + q * K3_THREADS, n16 - 1)]; };
            auto astore = [&](int q, const uint4& v) {
                if (tid + q * K3_THREADS < n16) reinterpret_cast<uint4*>(As)[tid + q * K3_THREADS] = v;
            };
            av0 = aload(0);
            av1 = aload(1);
            av2 = aload(2);
            av3 = aload(3);
            av4 = aload(4);
            // the previous pair's epilogue has finished reading As (DL: an
            // LDS-only barrier, so the tiles streaming in stay in flight)
            if constexpr (DL) lds_barrier(); else __syncthreads();
            astore(0, av0);
            astore(1, av1);
            astore(2, av2);
            astore(3, av3);
            astore(4, av4);
            if constexpr (X) {  // the low part: a second round
                av0 = aload(5);
                av1 = aload(6);
                av2 = aload(7);
                av3 = aload(8);
                av4 = aload(9);
                astore(5, av0);
                astore(6, av1);
                astore(7, av2);
                astore(8, av3);
                astore(9, av4);
            }
            if constexpr (DL) {
                lds_barrier();
            } else {
                __threadfence_block();
                __syncthreads();
            }
        } else {
            __syncthreads();  // the previous pair's epilogue has finished reading As
            int32_t te, tt;
            float sg;
            epoch_thread_sign(P.epoch, 2 * pair, P.nreuse, &te, &tt, &sg);
            const uint64_t seed = noise_seed(P.key, te, tt);
            const int32_t segs = P.segs, sl = r / segs;
            for (int32_t u = tid; u < (a + b) * segs; u += K3_THREADS) {
                const int32_t j = u / segs, c0 = (u - j * segs) * sl;
                uint64_t s = row_start_state(seed, u, P.jump);
                const StreamRow sr(P, j);
                float* rp = P.rec ? P.rec + ((size_t)pi * r + c0) * (a + b) + j : nullptr;
                if (sr.in_side) {
                    uint16_t* dst = slot + sr.row;
                    bm_rec_run(s, sl, ctx, rp, a + b,
                               [&](int32_t c, float v) { dst[(size_t)(c0 + c) * kp] = f2bf(v * sr.scale); });
                } else {
                    uint16_t* dst = As + (size_t)sr.row * lay.apitch;
                    bm_rec_run(s, sl, ctx, rp, a + b,
                               [&](int32_t c, float v) { dst[swap23(c0 + c)] = f2bf(v * sr.scale); });
                    if (c0 + sl == r)  // r is a multiple of 16: the padding maps onto itself
                        for (int32_t c = r; c < rp32; ++c) dst[c] = 0;
                }
            }
            __threadfence_block();
            __syncthreads();
        }

        // Bit rows of the block starting at L (of a pair ending at row rhi):
        // thread t loads words t % 2 + 2q of block row t / 2.
        // The loads are unconditional (rows past the pair's end read its last
        // row, words past the row its last word) and the result is masked when
        // stored, so nothing waits for them before xbits_store.
        bool xs_ok = false;
        auto xbits_load = [&](const RowCursor& cr, int64_t L, int64_t rhi, uint64_t (&v)[K3_XPF]) {
            const int32_t nv = (int32_t)min<int64_t>(rhi - L, K3_RB);
            xs_ok = xs_row < nv;
            int32_t m, qq;
            cr.at(min(xs_row, nv - 1), R, &m, &qq);
            const uint64_t* src = static_cast<const uint64_t*>(P.x) +
                                  k2_phys(m, qq, P.rpm, P.T, P.x_stride, P.x_plane);
#pragma unroll
            for (int q = 0; q < K3_XPF; ++q) v[q] = src[min(xs_w + 2 * q, nkt - 1)];
        };
        // Every loaded register is read here on every path (the empty asm),
        // so the compiler sees no load in flight across the block loop's back
        // edge and does not wait for all memory at the next block's start.
        auto consume = [](const uint64_t (&v)[K3_XPF]) {
#pragma unroll
            for (int q = 0; q < K3_XPF; ++q) asm volatile("" ::"v"(v[q]));
        };
        auto xbits_store = [&](const uint64_t (&v)[K3_XPF]) {
#pragma unroll
            for (int q = 0; q < K3_XPF; ++q) {
                const int32_t w = xs_w + 2 * q;
                if (w < nkt) Xbits[xs_row * nkt + w] = xs_ok ? v[q] : 0ull;
            }
            consume(v);
        };
        // Packed layout (P.x_packed): the block's nv rows are the nv * nkt
        // words from L * nkt on, stored to Xbits as they lie.  Wave w moves the
        // 16-byte chunks of its own rows 32w .. 32w + 31 (16 nkt chunks; lane l
        // takes chunks l + 64 q), so that with resident tiles each wave still
        // reads only the bit rows it staged.  Loads are clamped to the valid
        // words; words past them are stored as zero.  (The same registers as
        // the gathered form: chunk q in v[2q], v[2q + 1].)
        int32_t xp_nw = 0;  // valid words of the block being staged
        const int32_t xp_c0 = 16 * nkt * wave;  // this wave's first chunk
        auto xbits_load_packed = [&](int64_t L, int64_t rhi, uint64_t (&v)[K3_XPF]) {
            const int32_t nv = (int32_t)min<int64_t>(rhi - L, K3_RB);
            xp_nw = nv * nkt;
            const uint4* src = reinterpret_cast<const uint4*>(static_cast<const uint64_t*>(P.x) + L * nkt);
            const int32_t cmax = (xp_nw - 1) >> 1;
#pragma unroll
            for (int q = 0; q < K3_XPF / 2; ++q) {
                const uint4 u = src[min(xp_c0 + lane + 64 * q, cmax)];
                v[2 * q] = ((uint64_t)u.y << 32) | u.x;
                v[2 * q + 1] = ((uint64_t)u.w << 32) | u.z;
            }
        };
        auto xbits_store_packed = [&](const uint64_t (&v)[K3_XPF]) {
#pragma unroll
            for (int q = 0; q < K3_XPF / 2; ++q) {
                const int32_t cl = lane + 64 * q, c = xp_c0 + cl;
                if (cl < 16 * nkt) {
                    const uint64_t lo = 2 * c < xp_nw ? v[2 * q] : 0ull;
                    const uint64_t hi = 2 * c + 1 < xp_nw ? v[2 * q + 1] : 0ull;
                    reinterpret_cast<uint4*>(Xbits)[c] =
                        make_uint4((uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32));
                }
            }
            consume(v);
        };

        // ---- 2./3. row blocks ----------------------------------------------------
        uint4 pf0, pf1, pf2, pf3;
        uint64_t xpf[K3_XPF];
        // (member, row) of a block's first row: a pair's rows start at row 0
        // of its first member, and a block's cursor is the previous one's
        // advanced by K3_RB rows (no 64-bit division per block).
        auto advance = [&](RowCursor c) {
            c.q0 += K3_RB;
            if (c.q0 >= R) {
                const int32_t d = c.q0 / R;
                c.m0 += d;
                c.q0 -= d * R;
            }
            return c;
        };
        RowCursor cur_rows = unit_cursor(pi, part);
        for (int64_t L0 = row_lo; L0 < row_hi; L0 += K3_RB) {
            const bool first = L0 == row_lo;
            const bool has_next = L0 + K3_RB < row_hi;
            if (!first) cur_rows = advance(cur_rows);
            const int32_t nvalid = (int32_t)min<int64_t>(row_hi - L0, K3_RB);
            // DL: this wave's tile source for this block and for the next
            // block (the next unit's first block after the unit's last)
            const uint16_t* blk_src = dl_src;
            const uint16_t* nblk_src = has_next ? dl_src : dl_src_next;
            if (first && !xready) {
                if (P.x_packed) {
                    xbits_load_packed(L0, row_hi, xpf);
                    xbits_store_packed(xpf);
                } else {
                    xbits_load(cur_rows, L0, row_hi, xpf);
                    xbits_store(xpf);
                }
            }
            if constexpr (DL) {
                // the stream's first two tiles; later blocks' tiles were issued
                // during the previous block's last two tiles
                if (!dl_primed) {
                    // X: tile 1 into the other of the two buffers (a block has
                    // at least two stream tiles)
                    dl_issue_t(blk_src, 0, dl_cb);
                    dl_issue_t(blk_src, 1, dl_cb + 1 == NBUF ? 0 : dl_cb + 1);
                    wait_vmcnt<4>();
                    dl_primed = true;
                }
            } else if (first) {
                K3_TILE_LOAD(0);
                K3_TILE_STORE(0);
                if (resident && nkt > 1) {
                    K3_TILE_LOAD(1);
                    K3_TILE_STORE(1);
                }
            }
            // resident tiles: after a pair's first block each wave reads only the
            // bit rows it staged itself (thread t stages row t / 2), so waves order
            // their own LDS accesses and run their blocks out of step
            if (!resident || first)
                lds_barrier();
            else
                wave_lds_sync();
            if (!DL && nkt > 1 && !resident) K3_TILE_LOAD(1);

            f32x16 accW[4], accB[4];
            const uint32_t* xw = Xbits32 + (wrow0 + xrow) * (2 * nkt);
            // The K loop.  A K tile is four k-steps of 16 (this lane's 8 k at
            // 16 ks + 8 hl), each an x expansion and 8 MFMAs on 8 operand
            // fragments.  The fragment reads are rolled: right after the MFMA
            // that consumes fragment j of a step, fragment j of the next step is
            // read into the same registers, so each read has the following seven
            // MFMAs to land.  Across a tile boundary (non-resident tiles) the
            // barrier that publishes the next tile comes before the tile's last
            // step, whose MFMAs then cover the next tile's first reads.  ZERO:
            // the block's first tile, whose first step starts from the zero
            // operand instead of clearing 128 accumulator registers.
            u16x8 fr[8];
            // Fragment base of LDS tile buffer `bsel` at k-step ks; DL buffers
            // are unpadded and XOR-swizzled (chunk 2 ks + hl of column c at
            // slot (2 ks + hl) ^ ((c / 2) & 7); c / 2 mod 8 is lc / 2 mod 8 for
            // every staged column this lane reads).
            const int32_t dl_u = hl ^ ((lc >> 1) & 7);
            auto frag_ptr = [&](int32_t bsel, int ks) -> const uint16_t* {
                if constexpr (DL)
                    return WB + bsel * K3_DLTILE + lc * K2_BK + (((2 * ks) ^ dl_u) << 3);
                else
                    return WB + bsel * (K2_COLS * K2_TP) + lc * K2_TP + hl * 8 + 16 * ks;
            };
            auto frag_off = [](int j) {
                return ((j < 4 ? 0 : K2_NMAX) + 32 * (j & 3)) * (DL ? K2_BK : K2_TP);
            };
            {
                const uint16_t* tb = frag_ptr(DL ? dl_cb : 0, 0);
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (j >= WT && j < 4)
                        fr[j] = u16x8{};
                    else
                        fr[j] = lds_u16x8(tb + frag_off(j));
            }
            uint32_t xw0 = xw[0], xw1 = xw[1];
            // One step: its 8 MFMAs, each followed by the read of the same
            // fragment of the step at `nxt`.
            auto step = [&](uint32_t w, auto kc, auto zc, const uint16_t* nxt) {
                constexpr int ks = decltype(kc)::value;
                constexpr bool z = decltype(zc)::value;
                const uint32_t xbyte = (w >> (8 * ((ks & 1) * 2 + hl))) & 0xffu;
                const u16x8 xa = X ? expand_bits_f16(xbyte) : expand_bits(xbyte);
                auto mma = [](const u16x8& p, const u16x8& q, const f32x16& c) {
                    return X ? mfma32_f16(p, q, c) : mfma32_bf16(p, q, c);
                };
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    if (j >= WT && j < 4) continue;
                    if (j < 4)
                        accW[j] = mma(xa, fr[j], z ? f32x16{} : accW[j]);
                    else
                        accB[j - 4] = mma(fr[j], xa, z ? f32x16{} : accB[j - 4]);
                    fr[j] = lds_u16x8(nxt + frag_off(j));
                    __builtin_amdgcn_sched_barrier(0);
                }
            };
            // Tile kt sits in LDS buffer kt & 1 (DL: dl_cb); the next one is
            // staged into the other buffer during this one (unless the tiles are
            // resident; DL: the tile two ahead in the stream is issued and the
            // next one waited for).  The last tile's last step re-reads its own
            // first fragments (no branch around the reads; the values are unused).
            const bool dl_next_pair = !has_next && more_pairs;
            const int32_t ntb = DL ? nt : nkt;  // tiles of this block's K loop
            // X: stream tile t (t >= ntb: the next block's, or the next unit's
            // pair's, tile t - ntb) into buffer buf, issued right after the
            // barrier that frees buf (the one after the last reads of the
            // tile it held), so a transfer has four k-steps to land.
            auto dl_issue_ahead = [&](int32_t t, int32_t buf) {
                const uint16_t* src2 = blk_src;
                bool v = true;
                if (t >= ntb) {
                    t -= ntb;
                    src2 = nblk_src;
                    v = has_next || dl_next_pair;
                }
                if (v) dl_issue_t(src2, t, buf);
            };
            bool dl_v2 = false;  // DL: this tile issued the stream's tile DIST ahead
            // DL: tile DIST ahead in flight; the one just issued may remain so
            // (DIST 2), or every transfer has landed (X: the only one in
            // flight is the tile the barrier publishes)
            auto dl_wait = [&]() {
                if (DIST == 2 && dl_v2)
                    wait_vmcnt<4>();
                else
                    wait_vmcnt<0>();
            };
            auto tile = [&](int32_t kt, auto zc) {
                const bool more = kt + 1 < ntb;
                const int32_t kn = more ? kt + 1 : kt;
                const int32_t kw = X ? kn >> 1 : kn;  // x word of tile kn
                const int32_t cb = DL ? dl_cb : (kt & 1);
                const int32_t nb = DL ? (dl_cb + 1 == NBUF ? 0 : dl_cb + 1) : ((kt + 1) & 1);
                const uint32_t w0 = xw0, w1 = xw1;
                step(w0, std::integral_constant<int, 0>{}, zc, frag_ptr(cb, 1));
                step(w0, std::integral_constant<int, 1>{}, std::false_type{}, frag_ptr(cb, 2));
                if constexpr (DL) {
                    if constexpr (!EARLY) {
                        int32_t t2 = kt + DIST;
                        const uint16_t* src2 = dl_src;
                        dl_v2 = true;
                        if (t2 >= ntb) {
                            t2 -= ntb;
                            if (!has_next) {
                                src2 = dl_src_next;
                                dl_v2 = dl_next_pair;
                            }
                        }
                        if (dl_v2) dl_issue_t(src2, t2, nb + 1 == NBUF ? 0 : nb + 1);
                    }
                } else if (more && !resident) {
                    K3_TILE_STORE((kt + 1) & 1);
                    if (kt + 2 < nkt) K3_TILE_LOAD(kt + 2);
                }
                step(w1, std::integral_constant<int, 2>{}, std::false_type{}, frag_ptr(cb, 3));
                if (more && !resident) {
                    if constexpr (DL) dl_wait();  // tile kt + 1 has landed
                    lds_barrier();
                    if constexpr (EARLY) dl_issue_ahead(kt + 2, cb);
                }
                xw0 = xw[2 * kw];
                xw1 = xw[2 * kw + 1];
                step(w1, std::integral_constant<int, 3>{}, std::false_type{}, frag_ptr(more ? nb : cb, 0));
                if constexpr (DL) dl_cb = nb;
            };
            tile(0, std::true_type{});
            for (int32_t kt = 1; kt < ntb; ++kt) tile(kt, std::false_type{});
            // resident tiles: the epilogue restages only this wave's bit rows.
            // DL: the next block's first tile has landed before this barrier.
            if (!resident || nkt == 1) {
                if constexpr (DL) dl_wait();
                lds_barrier();
                // X: the next block's second tile, into the last tile's buffer
                if constexpr (EARLY) dl_issue_ahead(ntb + 1, dl_cb == 0 ? 1 : 0);
            } else {
                wave_lds_sync();
            }

            const bool next_pair = !has_next && more_pairs;
            // sign * xB as bf16: lane l holds rank columns 32j + 8g + 4hl + v of
            // the row at MFMA position lc (the row its x operand came from).
            // X: the same as fp16 high and low parts (xbf, xlo).
            uint32_t xbf[4][4][2];
            uint32_t xlo[4][4][2];
            {
                int32_t m, q;
                cur_rows.at(wrow0 + xrow, R, &m, &q);
                // odd members carry -A: negate after rounding (RNE is symmetric)
                const uint32_t sgn = ((P.tid_lo + m) & 1) ? 0x80008000u : 0u;
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        if constexpr (X) {
                            split_f16x2(accB[j][4 * g], accB[j][4 * g + 1], &xbf[j][g][0], &xlo[j][g][0]);
                            split_f16x2(accB[j][4 * g + 2], accB[j][4 * g + 3], &xbf[j][g][1], &xlo[j][g][1]);
                            xlo[j][g][0] ^= sgn;
                            xlo[j][g][1] ^= sgn;
                        } else {
                            xbf[j][g][0] = pack_bf16x2(accB[j][4 * g], accB[j][4 * g + 1]);
                            xbf[j][g][1] = pack_bf16x2(accB[j][4 * g + 2], accB[j][4 * g + 3]);
                        }
                        xbf[j][g][0] ^= sgn;
                        xbf[j][g][1] ^= sgn;
                    }
            }
            // accW += (sign xB) A^T over K = r in steps of 16: step (j, t) gives
            // k-group hl the rank columns 32j + 16t + 4hl + {0..3, 8..11}, stored
            // (swap23) as the 8 columns 32j + 16t + 8hl.
            const uint16_t* abase = As + (size_t)lc * K3_AP + 8 * hl;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (32 * j >= rp32) break;
                // the 16 A reads of this rank tile, then its 8 MFMAs (absent
                // output tiles, 32 jo >= a, read row lc of tile 0; their columns
                // are never stored)
                // X: (xB)_hi A_hi + (xB)_lo A_hi, then (xB)_hi A_lo (A's low part
                // at row a of the LDS block)
#pragma unroll
                for (int part = 0; part < (X ? 2 : 1); ++part) {
                    uint4 af[2][4];
#pragma unroll
                    for (int t = 0; t < 2; ++t)
#pragma unroll
                        for (int jo = 0; jo < WT; ++jo) {
                            const uint16_t* ap = abase + part * a * K3_AP +
                                                 (32 * jo < a ? 32 * jo * K3_AP : 0) + 32 * j + 16 * t;
                            af[t][jo] = *reinterpret_cast<const uint4*>(ap);
                        }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int t = 0; t < 2; ++t) {
                        const uint32_t d[4] = {xbf[j][2 * t][0], xbf[j][2 * t][1], xbf[j][2 * t + 1][0],
                                               xbf[j][2 * t + 1][1]};
                        const u16x8 xo = __builtin_bit_cast(u16x8, d);
#pragma unroll
                        for (int jo = 0; jo < WT; ++jo) {
                            if constexpr (X)
                                accW[jo] = mfma32_f16(xo, __builtin_bit_cast(u16x8, af[t][jo]), accW[jo]);
                            else
                                accW[jo] = mfma32_bf16(xo, __builtin_bit_cast(u16x8, af[t][jo]), accW[jo]);
                        }
                        if constexpr (X) {
                            if (part == 0) {
                                const uint32_t e[4] = {xlo[j][2 * t][0], xlo[j][2 * t][1],
                                                       xlo[j][2 * t + 1][0], xlo[j][2 * t + 1][1]};
                                const u16x8 xl = __builtin_bit_cast(u16x8, e);
#pragma unroll
                                for (int jo = 0; jo < WT; ++jo)
                                    accW[jo] = mfma32_f16(xl, __builtin_bit_cast(u16x8, af[t][jo]), accW[jo]);
                            }
                        }
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }

            // The next block's operands land during the LIF and the stores: its
            // bit rows (the next pair's first block after a pair's last one) and,
            // without DL, inside a pair, its first W/B tile.  Issued after the
            // second product: issued before it, the gathered rows stalled the
            // wave for about as long as the product takes, and the packed rows
            // (issued there) gained nothing while their registers spilled.
            // (Issued without branches: the last block of the last pair reloads
            // its own rows and tile, which are then not used.)
            {
                int64_t nlo = L0, nhi = row_hi;
                RowCursor ncr = cur_rows;
                if (has_next) {
                    nlo = L0 + K3_RB;
                    ncr = advance(cur_rows);
                } else if (next_pair) {
                    unit_rows(pi_n, part_n, &nlo, &nhi);
                    ncr = unit_cursor(pi_n, part_n);
                }
                if (P.x_packed)
                    xbits_load_packed(nlo, nhi, xpf);
                else
                    xbits_load(ncr, nlo, nhi, xpf);
                if (!DL && !resident) K3_TILE_LOAD(0);
            }

            // accW[jo][4g + v]: wave row 16 hl + 4g + v, column 32 jo + lc
            if constexpr (EPI == EPI_Y) {
#pragma unroll
                for (int g = 0; g < 4; ++g)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int32_t row = wrow0 + 16 * hl + 4 * g + v;
                        if (row >= nvalid) continue;
                        int32_t m, q;
                        cur_rows.at(row, R, &m, &q);
                        float* yrow = P.y + k2_phys(m, q, P.rpm, P.T, P.y_stride, P.y_plane);
#pragma unroll
                        for (int jo = 0; jo < WT; ++jo)
                            if (32 * jo + lc < a)
                                yrow[32 * jo + lc] = X ? accW[jo][4 * g + v] * (1.0f / K3_XSCALE)
                                                       : accW[jo][4 * g + v];
                    }
            } else {
                // LIF (snn.rs:53-97) along each lane's rows, v = 0 at t = 0.  The
                // reset keeps `charged` when no spike fired and gives 0 otherwise:
                // the reference's charged * (1 - spike) differs only in the sign
                // of a zero, which leaves every later `charged` (and spike) equal.
                float vm[4];
                int32_t cnt[4];
                uint32_t wlo[2] = {0, 0}, whi[2] = {0, 0};  // lane u: spike words of wave row u
                bool colok[4];
#pragma unroll
                for (int jo = 0; jo < 4; ++jo) colok[jo] = 32 * jo + lc < a;
                static_for<0, 16>([&](auto qc) {
                    constexpr int qq = decltype(qc)::value;  // 4g + v: time step qq % T
                    if constexpr (qq % LT == 0) {
#pragma unroll
                        for (int jo = 0; jo < 4; ++jo) {
                            vm[jo] = 0.0f;
                            cnt[jo] = 0;
                        }
                    }
                    uint64_t bal[4];
#pragma unroll
                    for (int jo = 0; jo < 4; ++jo) {
                        const float c = X ? accW[jo][qq] * (1.0f / K3_XSCALE) : accW[jo][qq];
                        const float charged = __fadd_rn(vm[jo], __fmul_rn(__fadd_rn(-vm[jo], c), P.leak));
                        const bool spike = charged >= P.v_th;
                        vm[jo] = spike ? 0.0f : charged;
                        if constexpr (RATE) cnt[jo] += spike ? 1 : 0;
                        if constexpr (SPK) bal[jo] = __builtin_amdgcn_ballot_w64(spike && colok[jo]);
                    }
                    if constexpr (RATE && qq % LT == LT - 1) {
                        const int32_t row = wrow0 + 16 * hl + qq;
                        if (P.cpl) {
                            // the counts' bit planes (0..LT needs log2(LT) + 1):
                            // ballot bit l is column 32 jo + l % 32 of the row of
                            // lane half l / 32, which lane 32 (l / 32) stores
                            constexpr int NPL = LT == 1 ? 1 : LT == 2 ? 2 : LT == 4 ? 3 : LT == 8 ? 4 : 5;
                            uint64_t pb[NPL][4];
#pragma unroll
                            for (int p = 0; p < NPL; ++p)
#pragma unroll
                                for (int jo = 0; jo < 4; ++jo)
                                    pb[p][jo] = __builtin_amdgcn_ballot_w64(((cnt[jo] >> p) & 1) && colok[jo]);
                            if (lc == 0 && row < nvalid) {
                                int32_t m, q;
                                cur_rows.at(row, R, &m, &q);
                                uint64_t* dst = P.cpl + ((int64_t)m * P.rpm + q / LT) * P.cpl_stride;
                                const int32_t words = (a + 63) >> 6;
#pragma unroll
                                for (int p = 0; p < NPL; ++p)
#pragma unroll
                                    for (int hh = 0; hh < 2; ++hh) {
                                        const uint64_t b0 = pb[p][2 * hh], b1 = pb[p][2 * hh + 1];
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
                            for (int jo = 0; jo < 4; ++jo)
                                if (colok[jo]) rp[32 * jo + lc] = (float)cnt[jo] * (1.0f / LT);
                        }
                    }
                    if constexpr (SPK) {
                        // ballot bit l: column 32 jo + l % 32 of wave row 16 (l / 32) + qq
#pragma unroll
                        for (int hh = 0; hh < 2; ++hh) {
                            const uint64_t b0 = bal[2 * hh], b1 = bal[2 * hh + 1];
                            put_lane<qq>(wlo[hh], whi[hh], (b0 & 0xffffffffull) | (b1 << 32));
                            put_lane<16 + qq>(wlo[hh], whi[hh], (b0 >> 32) | (b1 & 0xffffffff00000000ull));
                        }
                    }
                });
                if constexpr (SPK) {
                    if (lane < 32) {
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
            }
            if (!DL && has_next && !resident) K3_TILE_STORE(0);
            // stored also after the last block (the bit rows are then unused):
            // every path consumes the loads, so no load is left in flight
            // across the block loop's back edge
            if (P.x_packed)
                xbits_store_packed(xpf);
            else
                xbits_store(xpf);
            xready = next_pair;
        }
    }
#undef K3_TILE_LOAD
#undef K3_TILE_STORE
}

// Pair index range [lo, lo + cnt) of members [tid_lo, tid_lo + n).
inline int32_t pair_grid(const DeviceState* st, int32_t n_pairs) {
    return std::max(1, std::min(n_pairs, st->num_cus));
}

inline void pair_range(int32_t tid_lo, int32_t n, int32_t* lo, int32_t* cnt) {
    *lo = tid_lo / 2;
    *cnt = (tid_lo + n - 1) / 2 - *lo + 1;
}

}  // namespace hses
