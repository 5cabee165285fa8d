// tile_factors.h -- the rank-r factors of the members an output tile touches,
// generated from the noiser stream straight into LDS (shared by the
// small-rank and wide perturbed-forward kernels).
#pragma once
#include "linear_common.h"
#include "noise_dev.h"

namespace hses {

// Members [m_first, m_first + nm) of the tile: stream rows [f0, f0 + b) are
// the input-side operand, written as Bs[(member * r + c) * bpitch + k] in the
// MFMA type; rows [s0 + o0, s0 + o0 + ct) the output side for the tile's
// columns, written as As[(member * as_cols + o) * r + c] in fp32.  sign * sigma
// / sqrt(r) scales A of the parameter, the output side for do_mm (rows b..)
// and the input side for do_Tmm (rows a..).  Items are groups of P.rc stream
// rows (one jump each) spread over the block's threads.
template <int MATH>
__device__ __forceinline__ void gen_tile_factors(const LinParams& P, const NoiseCtx& ctx,
                                                 int32_t m_first, int32_t nm, int32_t o0,
                                                 int32_t ct, typename MathT<MATH>::T* Bs,
                                                 int32_t bpitch, float* As, int32_t as_cols) {
    const int32_t r = P.r, b = P.b, rc = P.rc;
    const int32_t f0 = P.tmm ? P.a : 0, s0 = P.tmm ? 0 : b;
    const float one = 1.0f;
    const int32_t qF0 = f0 / rc, qF1 = (f0 + b + rc - 1) / rc;
    const int32_t qS0 = (s0 + o0) / rc, qS1 = (s0 + o0 + ct + rc - 1) / rc;
    // the tile's output-side groups not already among the input side's
    const int32_t qX0 = P.tmm ? qS0 : max(qS0, qF1);
    const int32_t qX1 = P.tmm ? min(qS1, qF0) : qS1;
    const int32_t nF = qF1 - qF0;
    const int32_t per = nF + max(0, qX1 - qX0);
    for (int item = threadIdx.x; item < nm * per; item += blockDim.x) {
        const int32_t lm = item / per, qi = item % per;
        const int32_t q = qi < nF ? qF0 + qi : qX0 + (qi - nF);
        float sign;
        const uint64_t seed = member_seed(P.key, P.epoch, P.nreuse, P.tid_lo + m_first + lm, &sign);
        const float sc = sign * P.bs;
        const float fsc = P.tmm ? sc : one, ssc = P.tmm ? one : sc;
        uint64_t s = row_start_state(seed, q, P.jump);
        const int32_t rows_here = min(rc, P.a + b - q * rc);
        bm_run(s, rows_here * r, ctx, [&](int32_t i, float v) {
            const int32_t j = q * rc + i / r, c = i % r;
            if (j >= f0 && j < f0 + b) {
                Bs[(size_t)(lm * r + c) * bpitch + (j - f0)] = MathT<MATH>::cvt(v * fsc);
            } else {
                const int32_t o = j - s0 - o0;
                if (o >= 0 && o < ct) As[((size_t)lm * as_cols + o) * r + c] = v * ssc;
            }
        });
    }
}

}  // namespace hses
