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
//   2. for each 256-row block of the pair's rows: C = X [W^T | B] with bf16
//      MFMA.  Eight waves tile the block as 4 row groups x 2 column halves;
//      a wave owns 64 rows x (64 W columns + 64 B columns).  W/B tiles of 64 k
//      are double-buffered in LDS with the next tile prefetched into
//      registers during the current tile's MFMAs (one barrier per tile).
//      Bit-packed activations stay packed in LDS (one 64-bit word per row and
//      tile) and are expanded straight into MFMA operand registers;
//   3. epilogue: y = base + (sign_m xB) A^T with a second MFMA over K = r,
//      then either stored as fp32 or (fused LIF) transposed through LDS so
//      each lane holds one output column's whole time series, run through
//      the LIF update, and written as ballot-packed spike words and/or
//      spike rates; the fp32 currents never reach HBM.
// Rows inside a member are taken slot-major (q = s * T + t), so the T time
// steps of one (member, slot) are consecutive rows of one wave's row group.
// The (n, b, r) factor tensor is never materialised: at most one B per
// workgroup exists at any time.
//
// Two kernels share this structure.  k_linear_pair (below) takes any input
// format; k_pair_bits (further down) is the form for bit-packed input (the
// hidden layers of the SNN) and keeps its whole epilogue in registers.
#include "pair_bits.h"

namespace hses {

// W (a, b) fp32 -> (a, kp) bf16 with zero columns [b, kp); with tmm the
// parameter is stored (b, a) and is transposed on the way.
__global__ void k_w_to_bf16(const float* __restrict__ W, int32_t a, int32_t b, int32_t kp,
                            int32_t tmm, uint16_t* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)a * kp) return;
    const int32_t row = (int32_t)(i / kp), k = (int32_t)(i % kp);
    const int64_t src = tmm ? (int64_t)k * a + row : (int64_t)row * b + k;
    out[i] = k < b ? f2bf(W[src]) : (uint16_t)0;
}

// Factors of the pair kernels drawn ahead of their GEMM (the PRE kernels):
// one thread per (pair, stream row) continues its row of the pair's stream
// for r normals, keeps each raw normal in the factor record and its scaled
// bf16 value in the pair's operand image (PairImage).  Threads of
// output-side rows also zero the image's padding columns [b, kp) and their
// row's rank padding.  Lanes take consecutive stream rows, so for each rank
// column a wave's record stores and input-side image stores are contiguous
// runs.  Full occupancy (256-thread workgroups, no other work) keeps the
// VALU-bound generator at its rate.  X: the split image (PairImageX) instead,
// each value's fp16 high and low parts, A scaled by K3_XSCALE (the same
// values k_pair_image_x derives from the record).
constexpr int KG_THREADS = 256;
template <bool X = false>
__global__ __launch_bounds__(KG_THREADS) void k_pair_gen(const K2Args P) {
    __shared__ BmTables t;
    load_bm_tables(&t, P.tables);
    __syncthreads();
    const uint32_t rows = (uint32_t)(P.a + P.b);
    const uint32_t u = blockIdx.x * KG_THREADS + threadIdx.x;
    if (u >= (uint32_t)P.n_pairs * rows) return;
    const uint32_t pi = u / rows, j = u - pi * rows;
    const int32_t r = P.r, kp = (P.b + 63) / 64 * 64;
    int32_t te, tt;
    float sg;
    epoch_thread_sign(P.epoch, 2 * (P.pair_lo + (int32_t)pi), P.nreuse, &te, &tt, &sg);
    uint64_t s = row_start_state(noise_seed(P.key, te, tt), (int32_t)j, P.jump);
    const StreamRow sr(P, (int32_t)j);
    float* rp = P.rec + (size_t)pi * r * rows + j;
    const PairImage im(P.a, P.b, r);
    const PairImageX imx(P.a, P.b, r);
    uint16_t* img = P.bimg + (size_t)pi * (X ? imx.stride : im.stride);
    const size_t b_elems = X ? imx.b_elems : im.b_elems;
    // X: the low parts at `lo_off` elements after the high parts
    const size_t lo_off = sr.in_side ? imx.b_elems : imx.a_elems;
    // input side: element c at bp[c * kp]; output side: at bp[swap23(c)], where
    // swap23 keeps every aligned run of 4 rank columns contiguous, so an
    // output-side row stores each batch of 4 normals as one 8-byte write
    uint16_t* bp = sr.in_side ? img + sr.row : img + (X ? 2 : 1) * b_elems + (size_t)sr.row * (K2_NMAX + 8);
    // X: A (the output side) scaled by K3_XSCALE after the sigma scale
    const float xs = (X && !sr.in_side) ? K3_XSCALE : 1.0f;
    const NoiseCtx ctx{&t, P.log_exc, P.cos_exc};
    // no image (bimg NULL): the record alone
    const bool wimg = P.bimg != nullptr;
    // the record is read back by later kernels, long after this one:
    // non-temporal stores keep it from evicting the L2 lines of the kernels
    // that run beside the draw
    auto one = [&](int32_t c, float v) {
        __builtin_nontemporal_store(v, rp + (size_t)c * rows);
        if (!wimg) return;
        const size_t at = sr.in_side ? (size_t)c * kp : (size_t)swap23(c);
        if constexpr (X) {
            uint16_t hi, lo;
            split_f16(v * sr.scale * xs, &hi, &lo);
            bp[at] = hi;
            bp[at + lo_off] = lo;
        } else {
            bp[at] = f2bf(v * sr.scale);
        }
    };
    bm_run2(
        s, r, ctx,
        [&](int32_t c0, const float (&v)[4]) {
#pragma unroll
            for (int q = 0; q < 4; ++q) __builtin_nontemporal_store(v[q], rp + (size_t)(c0 + q) * rows);
            if (!wimg) return;
            if constexpr (X) {
                uint16_t hi[4], lo[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) split_f16(v[q] * sr.scale * xs, &hi[q], &lo[q]);
                if (sr.in_side) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        bp[(size_t)(c0 + q) * kp] = hi[q];
                        bp[(size_t)(c0 + q) * kp + lo_off] = lo[q];
                    }
                } else {
                    const uint2 wh{(uint32_t)hi[0] | ((uint32_t)hi[1] << 16),
                                   (uint32_t)hi[2] | ((uint32_t)hi[3] << 16)};
                    const uint2 wl{(uint32_t)lo[0] | ((uint32_t)lo[1] << 16),
                                   (uint32_t)lo[2] | ((uint32_t)lo[3] << 16)};
                    *reinterpret_cast<uint2*>(bp + swap23(c0)) = wh;
                    *reinterpret_cast<uint2*>(bp + swap23(c0) + lo_off) = wl;
                }
            } else if (sr.in_side) {
#pragma unroll
                for (int q = 0; q < 4; ++q) bp[(size_t)(c0 + q) * kp] = f2bf(v[q] * sr.scale);
            } else {
                const uint2 w{pack_bf16x2(v[0] * sr.scale, v[1] * sr.scale),
                              pack_bf16x2(v[2] * sr.scale, v[3] * sr.scale)};
                *reinterpret_cast<uint2*>(bp + swap23(c0)) = w;
            }
        },
        one);
    if (wimg && !sr.in_side) {
        for (int32_t c = r; c < ((r + 31) & ~31); ++c) {  // swap23 keeps 16-blocks
            bp[c] = 0;
            if constexpr (X) bp[c + lo_off] = 0;
        }
        for (int32_t k = P.b + sr.row; k < kp; k += P.a)
            for (int32_t c = 0; c < r; ++c) {
                img[(size_t)c * kp + k] = 0;
                if constexpr (X) img[b_elems + (size_t)c * kp + k] = 0;
            }
    }
}

void launch_w_to_bf16(const float* W, int32_t a, int32_t b, int32_t kp, int32_t tmm, uint16_t* out,
                      hipStream_t s) {
    const int64_t n = (int64_t)a * kp;
    hipLaunchKernelGGL(k_w_to_bf16, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, s, W, a, b, kp,
                       tmm, out);
}


// The split mode's W: (a, b) fp32 times K3_XSCALE as a high part (a, kp) and
// then a low part (a, kp), fp16, zero columns [b, kp).
// (do_mm only: W stored (a, b).)
__global__ void k_w_to_f16x(const float* __restrict__ W, int32_t a, int32_t b, int32_t kp,
                            uint16_t* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t n = (int64_t)a * kp;
    if (i >= n) return;
    const int32_t row = (int32_t)(i / kp), k = (int32_t)(i % kp);
    uint16_t hi = 0, lo = 0;
    if (k < b) split_f16(W[(int64_t)row * b + k] * K3_XSCALE, &hi, &lo);
    out[i] = hi;
    out[n + i] = lo;
}

// The split operand image (PairImageX) of every pair from the factor record
// (the raw normals; do_mm: stream rows [0, b) are B, [b, a + b) are A and
// carry the scale bs = sigma / sqrt(r) as the forward applies it, one fp32
// product).  Element e of a pair: e < r kp the B element (c, k) = (e / kp,
// e % kp), zero for k >= b; after that the A element (o, c) of a rows of
// r rounded up to 32, zero for c >= r.
__global__ void k_pair_image_x(const float* __restrict__ rec, int32_t a, int32_t b, int32_t r,
                               float bs, int32_t n_pairs, uint16_t* __restrict__ img) {
    const int32_t kp = (b + 63) / 64 * 64, rp32 = (r + 31) & ~31;
    const int64_t per = (int64_t)r * kp + (int64_t)a * rp32;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= per * n_pairs) return;
    const int64_t pi = i / per;
    const int64_t e = i - pi * per;
    const PairImageX im(a, b, r);
    uint16_t* dst = img + pi * im.stride;
    const float* rp = rec + pi * r * (int64_t)(a + b);
    uint16_t hi = 0, lo = 0;
    if (e < (int64_t)r * kp) {
        const int32_t c = (int32_t)(e / kp), k = (int32_t)(e % kp);
        if (k < b) split_f16(rp[(int64_t)c * (a + b) + k], &hi, &lo);
        dst[e] = hi;
        dst[im.b_elems + e] = lo;
    } else {
        const int64_t ea = e - (int64_t)r * kp;
        const int32_t o = (int32_t)(ea / rp32), c = (int32_t)(ea % rp32);
        if (c < r) split_f16(rp[(int64_t)c * (a + b) + b + o] * bs * K3_XSCALE, &hi, &lo);
        const size_t at = 2 * im.b_elems + (size_t)o * (K2_NMAX + 8) + swap23(c);
        dst[at] = hi;
        dst[at + im.a_elems] = lo;
    }
}



// Eight activations of one row from a dense format, as bf16.  With vec
// (strides that keep every 8-element group 16-byte aligned) a full group is
// two (f32) or one (bf16) 16-byte loads, issued unconditionally (rows outside
// the block address row 0) and masked after; otherwise, and for the group
// crossing b, element by element.
template <int XFMT>
__device__ __forceinline__ u16x8 dense_frag(const void* x, int64_t off, bool valid, int32_t k0,
                                            int32_t b, bool vec) {
    if constexpr (XFMT == HSES_FMT_F32 || XFMT == HSES_FMT_BF16) {
        if (vec && k0 + 8 <= b) {
            uint32_t d[4];
            if constexpr (XFMT == HSES_FMT_F32) {
                const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(x) + off + k0);
                const float4 lo = p[0], hi = p[1];
                d[0] = pack_bf16x2(lo.x, lo.y);
                d[1] = pack_bf16x2(lo.z, lo.w);
                d[2] = pack_bf16x2(hi.x, hi.y);
                d[3] = pack_bf16x2(hi.z, hi.w);
            } else {
                const uint4 q = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + off + k0);
                d[0] = q.x;
                d[1] = q.y;
                d[2] = q.z;
                d[3] = q.w;
            }
            const uint32_t m = valid ? 0xffffffffu : 0u;
            u16x8 v;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                v[2 * q] = (uint16_t)(d[q] & m);
                v[2 * q + 1] = (uint16_t)((d[q] & m) >> 16);
            }
            return v;
        }
    }
    u16x8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const bool ok = valid && k0 + e < b;
        if constexpr (XFMT == HSES_FMT_F32)
            v[e] = ok ? f2bf(static_cast<const float*>(x)[off + k0 + e]) : (uint16_t)0;
        else if constexpr (XFMT == HSES_FMT_BF16)
            v[e] = ok ? static_cast<const uint16_t*>(x)[off + k0 + e] : (uint16_t)0;
        else
            v[e] = ok ? f2bf((float)static_cast<const uint8_t*>(x)[off + k0 + e]) : (uint16_t)0;
    }
    return v;
}

// dense_frag's vector path in two parts, so that the loads of a fragment can
// be issued a step before it is used: the raw 16 or 32 bytes at (off + k0),
// then their bf16 form, masked when the row is absent (the same values).
template <int XFMT>
__device__ __forceinline__ void dense_raw(const void* x, int64_t off, int32_t k0, uint4 (&q)[2]) {
    if constexpr (XFMT == HSES_FMT_F32) {
        const uint4* p = reinterpret_cast<const uint4*>(static_cast<const float*>(x) + off + k0);
        q[0] = p[0];
        q[1] = p[1];
    } else {
        q[0] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + off + k0);
    }
}

template <int XFMT>
__device__ __forceinline__ u16x8 dense_cvt(const uint4 (&q)[2], bool valid) {
    uint32_t d[4];
    if constexpr (XFMT == HSES_FMT_F32) {
        d[0] = pack_bf16x2(__uint_as_float(q[0].x), __uint_as_float(q[0].y));
        d[1] = pack_bf16x2(__uint_as_float(q[0].z), __uint_as_float(q[0].w));
        d[2] = pack_bf16x2(__uint_as_float(q[1].x), __uint_as_float(q[1].y));
        d[3] = pack_bf16x2(__uint_as_float(q[1].z), __uint_as_float(q[1].w));
    } else {
        d[0] = q[0].x;
        d[1] = q[0].y;
        d[2] = q[0].z;
        d[3] = q[0].w;
    }
    const uint32_t m = valid ? 0xffffffffu : 0u;
    u16x8 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        v[2 * e] = (uint16_t)(d[e] & m);
        v[2 * e + 1] = (uint16_t)((d[e] & m) >> 16);
    }
    return v;
}

// Fused LIF on a wave's 64 rows x 64 output columns of currents (acc[i][j]:
// rows 16i + 4kg + v, columns 64h + 16j + li).  Per 16-row tile the currents
// go through a per-wave LDS scratch S[column][row] so lane l holds column
// 64h + l for 16 consecutive rows; the row group's rows are whole T-step
// series (T divides 64, slot-major rows), scanned in order with the update of
// hses_lif_scan (snn.rs:53-97) from v = 0.  Spikes of row u are ballot-packed
// into the 64-bit word of columns [64h, 64h + 64) held by lane u.  T is a
// template parameter so series boundaries are static.
template <int T>
__device__ __forceinline__ void lif_epilogue(const K2Args& P, const f32x4 (&acc)[4][8], float* S,
                                             const RowCursor& cur_rows, int wr, int h, int lane,
                                             int li, int kg, int32_t nvalid) {
    static_assert(T >= 1 && T <= 64 && (T & (T - 1)) == 0, "T must be a power of two <= 64");
    __syncthreads();  // every wave has finished reading XBs, which S aliases
    const bool col_ok = h * 64 + lane < P.a;
    uint32_t wlo = 0, whi = 0;  // lane u: spike word of row u (low / high half)
    float vm = 0.0f;
    int32_t cnt = 0;
    static_for<0, 4>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            *reinterpret_cast<f32x4*>(&S[(16 * j + li) * K2_LP + 4 * kg]) = acc[i][j];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        f32x4 c4[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) c4[q] = *reinterpret_cast<const f32x4*>(&S[lane * K2_LP + 4 * q]);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        static_for<0, 16>([&](auto uc) {
            constexpr int u = decltype(uc)::value;
            constexpr int rr = 16 * i + u;  // row inside the row group; time step rr % T
            if constexpr (rr % T == 0) {
                vm = 0.0f;
                cnt = 0;
            }
            const float c = c4[u >> 2][u & 3];
            // snn.rs:61-63: charged = v + ((-v) + c) * leak; each op rounds.
            const float charged = __fadd_rn(vm, __fmul_rn(__fadd_rn(-vm, c), P.leak));
            const bool spike = charged >= P.v_th;
            vm = __fmul_rn(charged, __fadd_rn(spike ? -1.0f : -0.0f, 1.0f));
            cnt += spike ? 1 : 0;
            put_lane<rr>(wlo, whi, __builtin_amdgcn_ballot_w64(spike && col_ok));
            if constexpr (rr % T == T - 1) {
                // spike rate of the series: count / T (exact: T is a power of two)
                const int32_t row = wr * 64 + rr;
                if (P.rate && row < nvalid && col_ok) {
                    int32_t m, q;
                    cur_rows.at(row, P.R, &m, &q);
                    P.rate[((int64_t)m * P.rpm + q / T) * P.rate_stride + h * 64 + lane] =
                        (float)cnt * (1.0f / T);
                }
            }
        });
    });
    if (P.spk && h * 64 < P.a) {
        const int32_t row = wr * 64 + lane;
        if (row < nvalid) {
            int32_t m, q;
            cur_rows.at(row, P.R, &m, &q);
            P.spk[k2_phys(m, q, P.rpm, T, P.spk_stride, P.spk_plane) + h] =
                ((uint64_t)whi << 32) | wlo;
        }
    }
}

// EPI: EPI_Y stores y; EPI_LIF + T (a power of two <= 64) runs the fused LIF.
// WJ: 16-column W tiles per wave (4 cover a <= 128; 1 suffices for a <= 16,
// e.g. a readout, and frees the registers of the other three).
// PRE: the factors were drawn ahead (k_pair_gen): A rows come from the
// record, B from the operand image, and nothing is generated.
template <int XFMT, int EPI, int LT = 1, int WJ = 4, bool PRE = false>
__global__ __launch_bounds__(K2_THREADS) void k_linear_pair(const K2Args P) {
    constexpr bool BITS = XFMT == HSES_FMT_BITS;
    static_assert(WJ >= 1 && WJ <= 4 && (EPI == EPI_Y || WJ == 4), "WJ < 4 only with EPI_Y");
    extern __shared__ __align__(16) unsigned char smem[];
    const K2Layout lay(P.r, P.b, BITS);
    BmTables* tabs = reinterpret_cast<BmTables*>(smem);
    uint16_t* As = reinterpret_cast<uint16_t*>(smem + lay.off_a);
    uint64_t* Xbits = reinterpret_cast<uint64_t*>(smem + lay.off_xbits);
    const uint32_t* Xbits32 = reinterpret_cast<const uint32_t*>(smem + lay.off_xbits);
    uint16_t* WB = reinterpret_cast<uint16_t*>(smem + lay.off_wb);  // [2][K2_COLS][K2_TP]
    uint16_t* XBs = WB;                                               // [K2_RB][apitch]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int li = lane & 15, kg = lane >> 4;
    const int wr = wave >> 1, h = wave & 1;
    const int32_t r = P.r, a = P.a, b = P.b, kp = lay.kp, nkt = lay.words, R = P.R;
    const int32_t rp32 = (r + 31) & ~31;
    const int32_t G = P.group;
    uint16_t* slots = PRE ? nullptr : P.slots + (size_t)blockIdx.x * G * r * kp;  // G slots of (r, kp)

    if constexpr (!PRE) {
        load_bm_tables(tabs, P.tables);
        // generation never writes k >= b: zero the slots' padding once
        for (int32_t i = tid; i < G * r * (kp - b); i += K2_THREADS) {
            const int32_t c = i / (kp - b), k = b + i % (kp - b);
            slots[(size_t)c * kp + k] = 0;
        }
        __threadfence_block();
        __syncthreads();
    }
    const NoiseCtx ctx{tabs, P.log_exc, P.cos_exc};

    // Tile loader: thread -> (staged column, 32-k half).  Columns [0, 128) are
    // W rows, [128, 256) rank columns of B; absent ones load a valid row and
    // are staged as zeros (a select, so the loads stay unconditional).
    const int lcol = tid >> 1, lk = (tid & 1) * 32;
    const bool lvalid = lcol < K2_NMAX ? lcol < a : lcol - K2_NMAX < r;
    const bool lw = lcol < K2_NMAX;
    const size_t loff = (size_t)(lw ? min(lcol, a - 1) : min(lcol - K2_NMAX, r - 1)) * kp + lk;
    const uint32_t lmask = lvalid ? 0xffffffffu : 0u;
    uint16_t* ldst = WB + lcol * K2_TP + lk;

    // The workgroup's pairs are blockIdx.x + i * gridDim.x; they are taken in
    // groups of G whose factors are generated together (small layers: a + b
    // stream rows of one pair leave most threads idle), pair g of a group
    // using slot g and A rows [g * a, g * a + a) of the LDS block.
    for (int32_t pi0 = blockIdx.x; pi0 < P.n_pairs; pi0 += G * (int32_t)gridDim.x) {
        const int32_t gcnt = min(G, (P.n_pairs - pi0 + (int32_t)gridDim.x - 1) / (int32_t)gridDim.x);

        // ---- 1. factors: A rows -> LDS (bf16, [o][c]); B rows -> slot ([c][k]) ----
        if constexpr (PRE) {
            // A^T of pair pi is rec[(pi r + c)(a + b) + aoff + o]: scale, round
            // and place it as the generation would have
            __syncthreads();  // the previous group's blocks have finished with As
            const int32_t per = r * a, aoff = P.tmm ? 0 : b;
            const float sc = P.tmm ? 1.0f : P.bs;
            for (int32_t i = tid; i < gcnt * per; i += K2_THREADS) {
                const int32_t g = i / per, e = i - g * per, c = e / a, o = e - c * a;
                const size_t pi = (size_t)(pi0 + g * (int32_t)gridDim.x);
                As[(size_t)(g * a + o) * lay.apitch + c] =
                    f2bf(P.rec[(pi * r + c) * (a + b) + aoff + o] * sc);
            }
            for (int32_t i = tid; i < gcnt * a * (rp32 - r); i += K2_THREADS)
                As[(size_t)(i / (rp32 - r)) * lay.apitch + r + i % (rp32 - r)] = 0;
            __threadfence_block();
            __syncthreads();
        } else {
            __syncthreads();  // the previous group's blocks have finished with As and the slots
            // Work units: segment of a stream row (P.segs segments of r / segs
            // normals) of one pair of the group.
            const int32_t segs = P.segs, sl = r / segs, upp = (a + b) * segs;
            for (int32_t u = tid; u < gcnt * upp; u += K2_THREADS) {
                const int32_t g = u / upp, uu = u - g * upp;
                const int32_t j = uu / segs, c0 = (uu - j * segs) * sl;
                int32_t te, tt;
                float sg;
                epoch_thread_sign(P.epoch, 2 * (P.pair_lo + pi0 + g * (int32_t)gridDim.x), P.nreuse,
                                  &te, &tt, &sg);
                uint64_t s = row_start_state(noise_seed(P.key, te, tt), uu, P.jump);
                const StreamRow sr(P, j);
                float* rp = P.rec ? P.rec + ((size_t)(pi0 + g * (int32_t)gridDim.x) * r + c0) * (a + b) + j
                                  : nullptr;
                if (sr.in_side) {
                    uint16_t* sg_ = slots + (size_t)g * r * kp + sr.row;
                    bm_rec_run(s, sl, ctx, rp, a + b,
                               [&](int32_t c, float v) { sg_[(size_t)(c0 + c) * kp] = f2bf(v * sr.scale); });
                } else {
                    uint16_t* arow = As + (size_t)(g * a + sr.row) * lay.apitch;
                    bm_rec_run(s, sl, ctx, rp, a + b,
                               [&](int32_t c, float v) { arow[c0 + c] = f2bf(v * sr.scale); });
                    if (c0 + sl == r)
                        for (int32_t c = r; c < rp32; ++c) arow[c] = 0;
                }
            }
            __threadfence_block();
            __syncthreads();
        }

    for (int32_t g = 0; g < gcnt; ++g) {
        const int32_t pi = pi0 + g * (int32_t)gridDim.x;
        const int32_t pair = P.pair_lo + pi;
        // Members of this pair inside the launch: m_lo .. m_hi (local indices).
        const int32_t m_even = 2 * pair - P.tid_lo;
        const int32_t m_lo = max(m_even, 0), m_hi = min(m_even + 1, P.n - 1);
        const int64_t row_lo = (int64_t)m_lo * R, row_hi = (int64_t)(m_hi + 1) * R;
        const uint16_t* lsrc =
            (lw ? P.wbf : PRE ? P.bimg + (size_t)pi * PairImage(a, b, r).stride : slots + (size_t)g * r * kp) + loff;
        const uint16_t* Ag = As + (size_t)g * a * lay.apitch;

        // ---- 2./3. row blocks ----------------------------------------------------
        for (int64_t L0 = row_lo; L0 < row_hi; L0 += K2_RB) {
            f32x4 acc[4][WJ + 4];  // [row group][W tiles, then 4 rank-column tiles of B]
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < WJ + 4; ++j) acc[i][j] = f32x4{0, 0, 0, 0};

            RowCursor cur_rows;
            cur_rows.m0 = (int32_t)(L0 / R);
            cur_rows.q0 = (int32_t)(L0 - (int64_t)cur_rows.m0 * R);
            const int32_t nvalid = (int32_t)min<int64_t>(row_hi - L0, K2_RB);
            int64_t xoff[4];
            bool xval[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int32_t row = wr * 64 + i * 16 + li;
                xval[i] = row < nvalid;
                int32_t m, q;
                cur_rows.at(row, R, &m, &q);
                xoff[i] = (!BITS && xval[i]) ? k2_phys(m, q, P.rpm, P.T, P.x_stride, P.x_plane) : 0;
            }
            if constexpr (BITS) {
                // the block's bit rows, one word per tile
                for (int32_t i = tid; i < K2_RB * nkt; i += K2_THREADS) {
                    const int32_t row = i / nkt, w = i - row * nkt;
                    int32_t m, q;
                    cur_rows.at(row, R, &m, &q);
                    Xbits[i] = row < nvalid
                                   ? static_cast<const uint64_t*>(P.x)[k2_phys(m, q, P.rpm, P.T, P.x_stride, P.x_plane) + w]
                                   : 0ull;
                }
            }
            // Dense x whose 8-element groups are 16-byte aligned and never
            // cross b, narrow outputs (one W tile per wave: the registers are
            // there): each sub-step's fragments are loaded one sub-step ahead
            // (the barriers below order LDS only, so these loads stay in flight).
            constexpr bool DENSE_VEC = (XFMT == HSES_FMT_F32 || XFMT == HSES_FMT_BF16) && WJ == 1;
            const bool xpre = DENSE_VEC && P.x_vec != 0 && b % K2_BK == 0;
            uint4 xr[4][2];
            if constexpr (DENSE_VEC) {
                if (xpre) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) dense_raw<XFMT>(P.x, xoff[i], kg * 8, xr[i]);
                }
            }
            // tile 0 -> buffer 0
            uint4 pf[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) pf[q] = reinterpret_cast<const uint4*>(lsrc)[q];
#pragma unroll
            for (int q = 0; q < 4; ++q) reinterpret_cast<uint4*>(ldst)[q] = mask4(pf[q], lmask);
            lds_barrier();

            for (int32_t kt = 0; kt < nkt; ++kt) {
                const int cur = kt & 1;
                const bool more = kt + 1 < nkt;
                if (more) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) pf[q] = reinterpret_cast<const uint4*>(lsrc + (kt + 1) * K2_BK)[q];
                }
                const uint16_t* tb = WB + cur * (K2_COLS * K2_TP);
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    u16x8 xa[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        if constexpr (BITS) {
                            const uint32_t w = Xbits32[(wr * 64 + i * 16 + li) * (2 * nkt) + 2 * kt + s];
                            xa[i] = expand_bits((w >> (8 * kg)) & 0xffu);
                        } else if (DENSE_VEC && xpre) {
                            xa[i] = dense_cvt<XFMT>(xr[i], xval[i]);
                        } else {
                            xa[i] = dense_frag<XFMT>(P.x, xoff[i], xval[i], kt * K2_BK + s * 32 + kg * 8, b,
                                                     P.x_vec != 0);
                        }
                    }
                    if constexpr (DENSE_VEC) {
                        const int32_t k1 = kt * K2_BK + (s + 1) * 32;  // the next sub-step's k
                        if (xpre && k1 < b) {
#pragma unroll
                            for (int i = 0; i < 4; ++i) dense_raw<XFMT>(P.x, xoff[i], k1 + kg * 8, xr[i]);
                        }
                    }
                    // absent columns are staged as zeros: no guards, straight-line MFMAs
#pragma unroll
                    for (int j = 0; j < WJ + 4; ++j) {
                        const int col = (j < WJ ? h * 64 + j * 16 : K2_NMAX + h * 64 + (j - WJ) * 16) + li;
                        const u16x8 bw = lds_u16x8(tb + col * K2_TP + s * 32 + kg * 8);
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[i][j] = mfma_bf16(xa[i], bw, acc[i][j]);
                    }
                }
                if (more) {
                    uint16_t* nb = ldst + (cur ^ 1) * (K2_COLS * K2_TP);
#pragma unroll
                    for (int q = 0; q < 4; ++q) reinterpret_cast<uint4*>(nb)[q] = mask4(pf[q], lmask);
                }
                lds_barrier();
            }

            // xB -> LDS as bf16 [row][c], sign of the row's member applied
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int row = wr * 64 + i * 16 + 4 * kg + v;
                    int32_t m, q;
                    cur_rows.at(row, R, &m, &q);
                    const float sgn = ((P.tid_lo + m) & 1) ? -1.0f : 1.0f;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int c = h * 64 + j * 16 + li;
                        if (h * 64 + j * 16 < r) XBs[row * lay.apitch + c] = f2bf(sgn * acc[i][WJ + j][v]);
                    }
                }
            if (rp32 != r) {  // K tail of the second product
                for (int32_t i = tid; i < K2_RB * 16; i += K2_THREADS)
                    XBs[(i >> 4) * lay.apitch + r + (i & 15)] = 0;
            }
            __syncthreads();
            // acc += (sign xB) A^T over K = r
            for (int32_t c0 = 0; c0 < rp32; c0 += 32) {
                u16x8 xf[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    xf[i] = lds_u16x8(&XBs[(wr * 64 + i * 16 + li) * lay.apitch + c0 + kg * 8]);
#pragma unroll
                for (int j = 0; j < WJ; ++j) {
                    if (h * 64 + j * 16 >= a) continue;
                    const u16x8 af = lds_u16x8(&Ag[(h * 64 + j * 16 + li) * lay.apitch + c0 + kg * 8]);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[i][j] = mfma_bf16(xf[i], af, acc[i][j]);
                }
            }
            if constexpr (EPI == EPI_Y) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int32_t row = wr * 64 + i * 16 + 4 * kg + v;
                        if (row >= nvalid) continue;
                        int32_t m, q;
                        cur_rows.at(row, R, &m, &q);
                        float* yrow = P.y + k2_phys(m, q, P.rpm, P.T, P.y_stride, P.y_plane);
#pragma unroll
                        for (int j = 0; j < WJ; ++j) {
                            const int col = h * 64 + j * 16 + li;
                            if (col < a) yrow[col] = acc[i][j][v];
                        }
                    }
            } else {
                lif_epilogue<LT>(P, acc, reinterpret_cast<float*>(WB) + wave * (64 * K2_LP), cur_rows,
                             wr, h, lane, li, kg, nvalid);
            }
            __syncthreads();  // XBs aliases the tile buffers; Xbits is restaged
        }
    }
    }
}


static bool pair_kernel_applies(const LinParams& P) {
    return (P.math == HSES_MATH_BF16 || P.math == HSES_MATH_F32X) && P.r >= 16 && P.r <= K2_NMAX && P.r % 16 == 0 &&
           P.a <= K2_NMAX;
}

// Pairs whose factors k_linear_pair generates together: as many as the A block
// of LDS (K2_NMAX rows) holds, at most 16.
static int32_t pair_group(int32_t a) { return std::max(1, std::min(K2_NMAX / a, 16)); }

// Segments per stream row for G pairs generated by `threads` threads: the
// fewest normals per thread, counting ~12 normals' worth of work for each
// segment's jump-ahead.
static int32_t gen_segs(int32_t G, int32_t a, int32_t b, int32_t r, int32_t threads) {
    int32_t best = 1;
    int64_t best_cost = INT64_MAX;
    for (int32_t segs = 1; segs <= 4; segs *= 2) {
        if (r % (segs * 8)) break;
        const int64_t units = (int64_t)G * (a + b) * segs;
        const int64_t cost = (units + threads - 1) / threads * (r / segs + 12);
        if (cost < best_cost) {
            best_cost = cost;
            best = segs;
        }
    }
    return best;
}

static size_t pair_workspace_bytes(int32_t slots, int32_t a, int32_t b, int32_t r) {
    const size_t kp = (size_t)(b + 63) / 64 * 64;
    return align16((size_t)a * kp * 2) + (size_t)slots * r * kp * 2;
}

// Sized for k_linear_pair's grouped slots, which k_pair_bits (one slot per
// workgroup) never exceeds.
// Also holds the split mode's W (high and low parts).
size_t linear_pair_workspace(const DeviceState* st, int32_t a, int32_t b, int32_t r, int32_t n) {
    int32_t lo, cnt;
    pair_range(0, n, &lo, &cnt);
    return std::max(pair_workspace_bytes(pair_grid(st, cnt + 1) * pair_group(a), a, b, r),
                    2 * pair_workspace_bytes(0, a, b, r));
}

// Every pair's factors of a launch drawn into the record and the B operand
// image (the PRE kernels' inputs).
int launch_pair_gen(LinParams& P, DeviceState* st, hipStream_t s, uint16_t* bimg, bool split) {
    if (P.r == 0 || !pair_kernel_applies(P)) return HSES_ERR_UNSUPPORTED;
    K2Args A{};
    pair_range(P.tid_lo, P.n, &A.pair_lo, &A.n_pairs);
    const int64_t units = (int64_t)A.n_pairs * (P.a + P.b);
    HSES_REQUIRE(units < (1ll << 31), "too many factor rows");
    int rc = get_jump_table(st, P.r, (int64_t)P.a + P.b, &A.jump);
    if (rc) return rc;
    A.key = P.key;
    A.tables = P.tables;
    A.log_exc = P.log_exc;
    A.cos_exc = P.cos_exc;
    A.a = P.a;
    A.b = P.b;
    A.r = P.r;
    A.epoch = P.epoch;
    A.nreuse = P.nreuse;
    A.bs = P.bs;
    A.tmm = P.tmm;
    A.rec = P.rec;
    A.bimg = bimg;
    const dim3 grid((uint32_t)((units + KG_THREADS - 1) / KG_THREADS));
    if (split)
        hipLaunchKernelGGL(k_pair_gen<true>, grid, dim3(KG_THREADS), 0, s, A);
    else
        hipLaunchKernelGGL(k_pair_gen<false>, grid, dim3(KG_THREADS), 0, s, A);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

int launch_pair_image_x(const float* rec, int32_t a, int32_t b, int32_t r, float bs, int32_t tid_lo,
                        int32_t n, uint16_t* img, hipStream_t s) {
    int32_t lo, cnt;
    pair_range(tid_lo, n, &lo, &cnt);
    const int32_t kp = (b + 63) / 64 * 64, rp32 = (r + 31) & ~31;
    const int64_t total = ((int64_t)r * kp + (int64_t)a * rp32) * cnt;
    if (total == 0) return HSES_OK;
    hipLaunchKernelGGL(k_pair_image_x, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, s, rec,
                       a, b, r, bs, cnt, img);
    HSES_CHECK_HIP(hipGetLastError());
    return HSES_OK;
}

size_t pair_image_x_bytes(int32_t a, int32_t b, int32_t r, int32_t tid_lo, int32_t n) {
    if (n < 1 || r < 1 || b < 1 || tid_lo < 0) return 0;
    int32_t lo, cnt;
    pair_range(tid_lo, n, &lo, &cnt);
    return (size_t)cnt * PairImageX(a, b, r).stride * 2;
}

size_t pair_image_bytes(int32_t a, int32_t b, int32_t r, int32_t tid_lo, int32_t n) {
    if (n < 1 || r < 1 || b < 1 || tid_lo < 0) return 0;
    int32_t lo, cnt;
    pair_range(tid_lo, n, &lo, &cnt);
    return (size_t)cnt * PairImage(a, b, r).stride * 2;
}

int launch_linear_pair(LinParams& P, DeviceState* st, hipStream_t s, void* work, size_t work_bytes,
                       const LifOut* lif, const uint16_t* bimg) {
    if (P.r == 0 || !pair_kernel_applies(P)) return HSES_ERR_UNSUPPORTED;
    const bool pre = bimg != nullptr;
    if (pre && !P.rec) return set_error(HSES_ERR_INVALID_ARG, "factors drawn ahead need the record");
    // the split (fp32-accurate) mode: drawn-ahead factors (a PairImageX image),
    // bit-packed x, do_mm, through the DL stream only
    const bool xm = P.math == HSES_MATH_F32X;
    if (xm && (!pre || P.x_fmt != HSES_FMT_BITS || P.tmm)) return HSES_ERR_UNSUPPORTED;
    if (lif && (P.n_time > 64 || (P.n_time & (P.n_time - 1)) != 0 || P.x_fmt != HSES_FMT_BITS))
        return HSES_ERR_UNSUPPORTED;
    const bool bits = P.x_fmt == HSES_FMT_BITS;
    // Bit-packed input with T <= 16 for the fused LIF: k_pair_bits.
    const bool v3 = bits && (!lif || P.n_time <= 16) && P.b <= 2 * K3_XPF * 64;
    if (lif && lif->cpl && !v3) return HSES_ERR_UNSUPPORTED;  // count planes: k_pair_bits only
    const K2Layout lay(P.r, P.b, bits);
    // factors drawn ahead and K of more than two tiles (any K in the split
    // mode): the DL tile stream
    const bool dl = v3 && pre && (xm || (P.b + 63) / 64 > 2) &&
                    K3Layout(P.r, P.b, true, xm).bytes <= st->max_lds;
    if (xm && !dl) return HSES_ERR_UNSUPPORTED;
    const K3Layout lay3(P.r, P.b, dl, xm);
    const size_t lds_bytes = v3 ? lay3.bytes : lay.bytes;
    const int threads = v3 ? K3_THREADS : K2_THREADS;
    if (lds_bytes > st->max_lds) return HSES_ERR_UNSUPPORTED;
    K2Args A{};
    pair_range(P.tid_lo, P.n, &A.pair_lo, &A.n_pairs);
    int32_t grid = pair_grid(st, A.n_pairs);
    // Pairs split over 4 workgroups of one XCD (the DL stream: drawn-ahead
    // factors, so no per-pair generation is repeated, and K of more than two
    // tiles; with resident tiles each part would restage them): every pair
    // full (both members), its blocks a multiple of 4, and the grid a
    // multiple of 32 workgroups.
    A.split = 1;
    if (dl && P.tid_lo % 2 == 0 && P.n % 2 == 0 && (2 * (int64_t)P.R) % (4 * K3_RB) == 0 &&
        st->num_cus % 32 == 0 && (int64_t)A.n_pairs * 4 >= st->num_cus) {
        A.split = 4;
        grid = st->num_cus;
    }
    A.group = v3 ? 1 : pair_group(P.a);
    const size_t need = xm ? 2 * pair_workspace_bytes(0, P.a, P.b, P.r)
                           : pair_workspace_bytes(pre ? 0 : grid * A.group, P.a, P.b, P.r);
    if (!work || work_bytes < need)
        return set_error(HSES_ERR_INVALID_ARG, "hses_perturbed_linear: workspace too small");
    uint16_t* wbf = static_cast<uint16_t*>(work);
    A.wbf = wbf;
    A.slots = reinterpret_cast<uint16_t*>(static_cast<char*>(work) + align16((size_t)P.a * lay.kp * 2));
    // Split each stream row into segs pieces (row length r / segs in the jump
    // table) when the group's a + b rows would leave threads idle.
    A.segs = gen_segs(A.group, P.a, P.b, P.r, threads);
    int rc = get_jump_table(st, P.r / A.segs, ((int64_t)P.a + P.b) * A.segs, &P.jump);
    if (rc) return rc;
    A.x = P.x;
    A.x_stride = P.x_stride;
    A.x_plane = P.x_plane;
    A.y = P.y;
    A.y_stride = P.y_stride;
    A.y_plane = P.y_plane;
    A.key = P.key;
    A.tables = P.tables;
    A.log_exc = P.log_exc;
    A.cos_exc = P.cos_exc;
    A.jump = P.jump;
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
    A.epoch = P.epoch;
    A.nreuse = P.nreuse;
    A.bs = P.bs;
    A.tmm = P.tmm;
    A.rec = P.rec;
    A.bimg = const_cast<uint16_t*>(bimg);
    {
        // 8 consecutive elements of a row start 16-byte aligned when the base,
        // the row stride and the plane stride all keep them so
        const int64_t g = P.x_fmt == HSES_FMT_F32 ? 4 : 8;  // elements per 16 bytes
        A.x_vec = (reinterpret_cast<uintptr_t>(P.x) % 16 == 0) && P.x_stride % g == 0 &&
                  P.x_plane % g == 0;
        const int64_t words = (P.b + 63) / 64;
        A.x_packed = bits && reinterpret_cast<uintptr_t>(P.x) % 16 == 0 && P.x_plane == words &&
                     P.x_stride == (int64_t)P.n_time * words && ((int64_t)P.R * words) % 2 == 0;
    }
    const int64_t wl = (int64_t)P.a * lay.kp;
    if (xm)
        hipLaunchKernelGGL(k_w_to_f16x, dim3((uint32_t)((wl + 255) / 256)), dim3(256), 0, s, P.W,
                           P.a, P.b, lay.kp, wbf);
    else
        hipLaunchKernelGGL(k_w_to_bf16, dim3((uint32_t)((wl + 255) / 256)), dim3(256), 0, s, P.W,
                           P.a, P.b, lay.kp, P.tmm, wbf);
    HSES_CHECK_HIP(hipGetLastError());
    auto launch = [&](auto kern) -> int {
        if (lds_bytes > 64 * 1024)
            HSES_CHECK_HIP(hipFuncSetAttribute((const void*)kern,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes));
        hipLaunchKernelGGL(kern, dim3(grid), dim3(threads), lds_bytes, s, A);
        HSES_CHECK_HIP(hipGetLastError());
        return HSES_OK;
    };
    if (v3) {
        auto by_pre = [&](auto pc, auto dc, auto xc) -> int {
            constexpr bool PR = decltype(pc)::value, D = decltype(dc)::value;
            constexpr bool XX = decltype(xc)::value;
            if (!lif) {
                // X with a <= 32 (the readout): one output tile
                if constexpr (XX)
                    if (P.a <= 32) return launch(k_pair_bits<EPI_Y, 1, false, false, PR, D, XX, 1>);
                return launch(k_pair_bits<EPI_Y, 1, false, false, PR, D, XX>);
            }
            const bool spk = lif->spk != nullptr, rate = lif->rate != nullptr || lif->cpl != nullptr;
            auto by_t = [&](auto sc, auto rc) -> int {
                constexpr bool S = decltype(sc)::value, Q = decltype(rc)::value;
                switch (P.n_time) {
                    case 1: return launch(k_pair_bits<EPI_LIF, 1, S, Q, PR, D, XX>);
                    case 2: return launch(k_pair_bits<EPI_LIF, 2, S, Q, PR, D, XX>);
                    case 4: return launch(k_pair_bits<EPI_LIF, 4, S, Q, PR, D, XX>);
                    case 8: return launch(k_pair_bits<EPI_LIF, 8, S, Q, PR, D, XX>);
                    default: return launch(k_pair_bits<EPI_LIF, 16, S, Q, PR, D, XX>);
                }
            };
            if (spk && rate) return by_t(std::true_type{}, std::true_type{});
            if (spk) return by_t(std::true_type{}, std::false_type{});
            return by_t(std::false_type{}, std::true_type{});
        };
        const std::true_type yes;
        const std::false_type no;
        if (xm) return by_pre(yes, yes, yes);
        if (dl) return by_pre(yes, yes, no);
        return pre ? by_pre(yes, no, no) : by_pre(no, no, no);
    }
    if (pre) {
        // dense input (the readout on spike rates) on the PRE form of k_linear_pair
        if (lif) return HSES_ERR_UNSUPPORTED;
        switch (P.x_fmt) {
            case HSES_FMT_F32:
                return P.a <= 16 ? launch(k_linear_pair<HSES_FMT_F32, EPI_Y, 1, 1, true>)
                                 : launch(k_linear_pair<HSES_FMT_F32, EPI_Y, 1, 4, true>);
            case HSES_FMT_BF16:
                return P.a <= 16 ? launch(k_linear_pair<HSES_FMT_BF16, EPI_Y, 1, 1, true>)
                                 : launch(k_linear_pair<HSES_FMT_BF16, EPI_Y, 1, 4, true>);
            default: return HSES_ERR_UNSUPPORTED;
        }
    }
    if (lif) {
        switch (P.n_time) {
            case 1: return launch(k_linear_pair<HSES_FMT_BITS, EPI_LIF, 1>);
            case 2: return launch(k_linear_pair<HSES_FMT_BITS, EPI_LIF, 2>);
            case 4: return launch(k_linear_pair<HSES_FMT_BITS, EPI_LIF, 4>);
            case 8: return launch(k_linear_pair<HSES_FMT_BITS, EPI_LIF, 8>);
            case 16: return launch(k_linear_pair<HSES_FMT_BITS, EPI_LIF, 16>);
            case 32: return launch(k_linear_pair<HSES_FMT_BITS, EPI_LIF, 32>);
            default: return launch(k_linear_pair<HSES_FMT_BITS, EPI_LIF, 64>);
        }
    }
    switch (P.x_fmt) {
        case HSES_FMT_F32:
            return P.a <= 16 ? launch(k_linear_pair<HSES_FMT_F32, EPI_Y, 1, 1>)
                             : launch(k_linear_pair<HSES_FMT_F32, EPI_Y>);
        case HSES_FMT_BF16:
            return P.a <= 16 ? launch(k_linear_pair<HSES_FMT_BF16, EPI_Y, 1, 1>)
                             : launch(k_linear_pair<HSES_FMT_BF16, EPI_Y>);
        default: return launch(k_linear_pair<HSES_FMT_BITS, EPI_Y>);
    }
}

}  // namespace hses
