// bm_tables.cpp -- host construction of the exact Box-Muller tables.
//
// The device evaluates log/cos with the f64 routines of bm_exact.h and needs:
//   * the small interpolation tables (log: 1/c and -log(1/c) per subinterval;
//     cos: cos, sin and a two-part angle per grid point);
//   * per-input exception bitmaps: bit k is set where glibc's logf/cosf differ
//     from the f32 rounding of the f64 routine;
//   * per-bucket danger window half-widths t (in 2^-29 f32 ulp) so that every
//     exception satisfies in_danger(y, t).
// glibc is the parity target because the reference's f32::ln / f32::cos lower
// to glibc logf / cosf on linux-gnu (noiser.rs:470-477).
#include <math.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <string>
#include <thread>
#include <vector>

#include "runtime.h"

namespace hses {

namespace {

void build_small(BmTables* t) {
    // log: 128 subintervals of the bit window [0.75f, 1.5f).
    for (int i = 0; i < kLogTab; ++i) {
        long double lo, w;
        if (i < 64) {
            lo = 0.75L + (long double)i * 0x1p-8L;
            w = 0x1p-8L;
        } else {
            lo = 1.0L + (long double)(i - 64) * 0x1p-7L;
            w = 0x1p-7L;
        }
        if (i == 63 || i == 64) {
            // z - 1 is exact next to 1: keep the full relative precision of log1p.
            t->log_invc[i] = 1.0;
            t->log_logc[i] = 0.0;
            continue;
        }
        const long double c = lo + w / 2;
        const double invc = (double)(1.0L / c);
        t->log_invc[i] = invc;
        t->log_logc[i] = (double)(-logl((long double)invc));
    }
    // cos: grid theta_j = j * 2pi / 64 with exact values at the quadrant points.
    const long double pi = 3.141592653589793238462643383279502884L;
    for (int j = 0; j <= kCosTab; ++j) {
        const long double th = (long double)j * 2.0L * pi / (long double)kCosTab;
        const double hi = (double)th;
        t->cos_thi[j] = hi;
        t->cos_tlo[j] = (double)(th - (long double)hi);
        double c = (double)cosl(th), s = (double)sinl(th);
        switch (j) {
            case 0: c = 1.0; s = 0.0; break;
            case 16: c = 0.0; s = 1.0; break;
            case 32: c = -1.0; s = 0.0; break;
            case 48: c = 0.0; s = -1.0; break;
            case 64: c = 1.0; s = 0.0; break;
            default: break;
        }
        t->cos_c[j] = c;
        t->cos_s[j] = s;
    }
}

struct Exc {
    uint32_t k;
    uint32_t dist;  // |R - 2^28|: distance to the rounding midpoint in 2^-29 ulp
};

// Evaluate one function over a slice of unit indices.  kind 0 = log, 1 = cos.
void scan_slice(const BmTables* t, int kind, uint32_t k_lo, uint32_t k_hi, std::vector<Exc>* exc,
                std::string* err) {
    for (uint32_t k = k_lo; k < k_hi; ++k) {
        double y;
        float ref;
        if (kind == 0) {
            const float x = log_arg(k);  // k == 0: the clamped 1e-9f
            y = log_f64(x, t->log_invc, t->log_logc);
            ref = logf(x);
        } else {
            const float th = cos_arg(k);
            y = cos_f64(th, k, t->cos_c, t->cos_s, t->cos_thi, t->cos_tlo);
            ref = cosf(th);
        }
        const float f = (float)y;
        if (f2u(ref) == f2u(f)) continue;
        const float g = other_candidate(f, rem29(y));
        if (f2u(ref) != f2u(g)) {
            char buf[160];
            snprintf(buf, sizeof buf,
                     "%s exception at k=%u is not the midpoint neighbour (ref %a, f %a, g %a)",
                     kind == 0 ? "log" : "cos", k, (double)ref, (double)f, (double)g);
            *err = buf;
            return;
        }
        const uint32_t R = rem29(y);
        exc->push_back({k, R >= 0x10000000u ? R - 0x10000000u : 0x10000000u - R});
    }
}

// Smallest window that puts every exception of a bucket in danger.
uint32_t bucket_t(const std::vector<Exc>& exc_in_bucket) {
    uint32_t t = 0;
    for (const Exc& x : exc_in_bucket) t = std::max(t, x.dist + 1u);
    return t;
}

}  // namespace

std::string build_bm_tables(HostBmTables* out, int nthreads) {
    build_small(&out->small);
    out->log_exc.assign(kBitmapAlloc, 0u);
    out->cos_exc.assign(kBitmapAlloc, 0u);
    if (nthreads < 1) nthreads = 1;
    for (int kind = 0; kind < 2; ++kind) {
        std::vector<std::vector<Exc>> parts(nthreads);
        std::vector<std::string> errs(nthreads);
        std::vector<std::thread> th;
        const uint32_t per = (kUnitCount + nthreads - 1) / nthreads;
        for (int i = 0; i < nthreads; ++i) {
            const uint32_t lo = std::min<uint64_t>((uint64_t)i * per, kUnitCount);
            const uint32_t hi = std::min<uint64_t>((uint64_t)(i + 1) * per, kUnitCount);
            th.emplace_back(scan_slice, &out->small, kind, lo, hi, &parts[i], &errs[i]);
        }
        for (auto& x : th) x.join();
        for (auto& e : errs)
            if (!e.empty()) return e;
        std::vector<std::vector<Exc>> by_bucket(kBuckets);
        uint32_t n = 0;
        std::vector<uint32_t>& bm = kind == 0 ? out->log_exc : out->cos_exc;
        for (auto& p : parts)
            for (const Exc& x : p) {
                bm[x.k >> 5] |= 1u << (x.k & 31);
                by_bucket[x.k >> kBucketShift].push_back(x);
                ++n;
            }
        DangerWin* tw = kind == 0 ? out->small.log_dw : out->small.cos_dw;
        for (int b = 0; b < kBuckets; ++b) {
            const uint32_t t = bucket_t(by_bucket[b]);
            if (t > 0x10000000u) return "danger window wider than half an ulp";
            tw[b] = DangerWin{0x10000000u - t, 2u * t};
            // every exception must test as dangerous with the bucket's window
            for (const Exc& x : by_bucket[b]) {
                const double y = kind == 0
                                      ? log_f64(log_arg(x.k), out->small.log_invc, out->small.log_logc)
                                      : cos_f64(cos_arg(x.k), x.k, out->small.cos_c, out->small.cos_s,
                                                out->small.cos_thi, out->small.cos_tlo);
                if (!in_danger(y, tw[b])) return "exception outside its danger window";
            }
        }
        if (kind == 0)
            out->n_log_exc = n;
        else
            out->n_cos_exc = n;
    }
    return std::string();
}

// ---------------------------------------------------------------------------
// GF(2) matrices for xorshift64 jump-ahead.
// ---------------------------------------------------------------------------

Gf2 gf2_identity() {
    Gf2 m;
    for (int i = 0; i < 64; ++i) m.c[i] = 1ull << i;
    return m;
}

Gf2 gf2_step() {
    Gf2 m;
    for (int i = 0; i < 64; ++i) m.c[i] = xs64(1ull << i);
    return m;
}

Gf2 gf2_mul(const Gf2& A, const Gf2& B) {
    Gf2 C;
    for (int i = 0; i < 64; ++i) C.c[i] = gf2_apply(A.c, B.c[i]);
    return C;
}

Gf2 gf2_pow(const Gf2& M, uint64_t n) {
    Gf2 r = gf2_identity(), b = M;
    while (n) {
        if (n & 1) r = gf2_mul(r, b);
        b = gf2_mul(b, b);
        n >>= 1;
    }
    return r;
}

}  // namespace hses
