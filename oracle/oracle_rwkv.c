/* oracle_rwkv.c -- CPU restatement of the RWKV-7 components of
 * burn_impl/hyperscalees-models/src/llm.rs (layer_norm, GroupNorm,
 * rwkv7_inner_loop, ChannelMixing).  Test infrastructure only, like oracle.c:
 * it is the checker of the GPU kernels, never on the product path.
 *
 * Reductions (means, dot products, matmuls) accumulate in f32 in ascending
 * index order, every operation rounded separately (built with
 * -ffp-contract=off); Burn's own reduction order is not observable, so those
 * sums are compared with tolerances, while the per-element arithmetic of the
 * recurrence follows the reference's operation order exactly. */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* llm.rs:66-83: (x - mean) / sqrt(var + eps) * w + b with var = E[x^2] - E[x]^2. */
void or_layer_norm(const float *x, int64_t rows, int32_t C, const float *w, const float *b,
                   float eps, float *y) {
    for (int64_t i = 0; i < rows; ++i) {
        const float *xr = x + i * C;
        float s = 0.0f, s2 = 0.0f;
        for (int32_t c = 0; c < C; ++c) {
            s = s + xr[c];
            s2 = s2 + xr[c] * xr[c];
        }
        const float mean = s / (float)C;
        const float var = s2 / (float)C - mean * mean;
        const float sd = sqrtf(var + eps);
        for (int32_t c = 0; c < C; ++c) y[i * C + c] = (xr[c] - mean) / sd * w[c] + b[c];
    }
}

/* llm.rs:97-150 (GroupNorm): x (n, C, L) (L = 1 for the rank-2 form), groups of
 * C/G channels x L positions normalised together, then gamma[c] * x + beta[c]. */
void or_group_norm(const float *x, int64_t n, int32_t C, int32_t L, int32_t G, const float *w,
                   const float *b, float eps, float *y) {
    const int32_t inner = C / G;
    const int64_t gsz = (int64_t)inner * L;
    for (int64_t i = 0; i < n; ++i)
        for (int32_t g = 0; g < G; ++g) {
            const float *xg = x + (i * C + (int64_t)g * inner) * L;
            float s = 0.0f, s2 = 0.0f;
            for (int64_t e = 0; e < gsz; ++e) {
                s = s + xg[e];
                s2 = s2 + xg[e] * xg[e];
            }
            const float mean = s / (float)gsz;
            const float var = s2 / (float)gsz - mean * mean;
            const float sd = sqrtf(var + eps);
            float *yg = y + (i * C + (int64_t)g * inner) * L;
            for (int64_t e = 0; e < gsz; ++e) {
                const int32_t c = g * inner + (int32_t)(e / L);
                yg[e] = w[c] * ((xg[e] - mean) / sd) + b[c];
            }
        }
}

/* llm.rs:235-300 (rwkv7_inner_loop).  r, w, k, v, a, b: (T, H, S); s0: (H, S, S);
 * new_starts: T bytes.  w -> exp(-exp(w)); per step: s = 0 on a new start,
 * sa = s @ a, s = s * w + v @ k + sa @ b, out[t] = s @ r, out_s = s of the last
 * step t < length (s0 when length == 0). */
void or_rwkv7_inner_loop(const float *r, const float *w, const float *k, const float *v,
                         const float *a, const float *b, const float *s0, int32_t T, int32_t H,
                         int32_t S, int32_t length, const uint8_t *new_starts, float *out,
                         float *out_s) {
    const int64_t hs = (int64_t)S * S;
    float *s = (float *)malloc(sizeof(float) * (size_t)(H * hs) + 4);
    float *sa = (float *)malloc(sizeof(float) * (size_t)S + 4);
    memcpy(s, s0, sizeof(float) * (size_t)(H * hs));
    memcpy(out_s, s0, sizeof(float) * (size_t)(H * hs));
    for (int32_t t = 0; t < T; ++t) {
        if (new_starts && new_starts[t]) memset(s, 0, sizeof(float) * (size_t)(H * hs));
        for (int32_t h = 0; h < H; ++h) {
            const int64_t o = ((int64_t)t * H + h) * S;
            float *sh = s + h * hs;
            for (int32_t i = 0; i < S; ++i) {
                float acc = 0.0f;
                for (int32_t j = 0; j < S; ++j) acc = acc + sh[i * S + j] * a[o + j];
                sa[i] = acc;
            }
            for (int32_t i = 0; i < S; ++i)
                for (int32_t j = 0; j < S; ++j) {
                    const float wd = expf(-expf(w[o + j]));
                    const float t1 = sh[i * S + j] * wd;
                    const float t2 = v[o + i] * k[o + j];
                    const float t4 = sa[i] * b[o + j];
                    sh[i * S + j] = (t1 + t2) + t4;
                }
            for (int32_t i = 0; i < S; ++i) {
                float acc = 0.0f;
                for (int32_t j = 0; j < S; ++j) acc = acc + sh[i * S + j] * r[o + j];
                out[o + i] = acc;
            }
        }
        if (t < length) memcpy(out_s, s, sizeof(float) * (size_t)(H * hs));
    }
    free(sa);
    free(s);
}

/* llm.rs:191-213 (ChannelMixing with plain linears): x (T, C), state (C),
 * x_k (C), Wk (F, C) key weight, Wv (C, F) value weight.
 * sx = [state, x[:-1]] (zero on new starts) - x; xk = x + sx * x_k;
 * out = relu(xk Wk^T)^2 Wv^T; last = x[length - 1]. */
void or_channel_mixing(const float *x, int32_t T, int32_t C, const float *state,
                       const float *x_k, const float *Wk, int32_t F, const float *Wv,
                       int32_t length, const uint8_t *new_starts, float *out, float *last) {
    float *xk = (float *)malloc(sizeof(float) * (size_t)T * C + 4);
    float *kk = (float *)malloc(sizeof(float) * (size_t)T * F + 4);
    for (int32_t t = 0; t < T; ++t)
        for (int32_t c = 0; c < C; ++c) {
            float prev = t == 0 ? state[c] : x[(int64_t)(t - 1) * C + c];
            if (new_starts && new_starts[t]) prev = 0.0f;
            const float sx = prev - x[(int64_t)t * C + c];
            xk[(int64_t)t * C + c] = x[(int64_t)t * C + c] + sx * x_k[c];
        }
    or_matmul_abt(xk, T, C, Wk, F, kk);
    for (int64_t e = 0; e < (int64_t)T * F; ++e) {
        const float z = kk[e] > 0.0f ? kk[e] : 0.0f;
        kk[e] = z * z;
    }
    or_matmul_abt(kk, T, F, Wv, C, out);
    memcpy(last, x + (int64_t)(length - 1) * C, sizeof(float) * (size_t)C);
    free(kk);
    free(xk);
}

/* y (m, n) = x (m, k) @ w (k, n): the Tmm forward (common.rs:156-159), f32 in ascending k. */
static void matmul_ab_f32(const float *x, int32_t m, int32_t k, const float *w, int32_t n, float *y) {
    for (int32_t i = 0; i < m; ++i)
        for (int32_t j = 0; j < n; ++j) {
            float acc = 0.0f;
            for (int32_t q = 0; q < k; ++q) acc = acc + x[(int64_t)i * k + q] * w[(int64_t)q * n + j];
            y[(int64_t)i * n + j] = acc;
        }
}

/* burn 0.21 (the reference's Cargo.toml:29; not vendored) defines
 * softplus(x, beta) = log(1 + exp(beta x)) / beta, called with beta = 1, and
 * sigmoid(x) = 1 / (1 + exp(-x)); its backends may round the latter differently
 * in the last place, inside the parity tolerance. */
static float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }
static float softplusf_(float x) { return logf(expf(x) + 1.0f); }

/* llm.rs:348-480 (TimeMixing::forward) for one sequence with plain weights.
 * x (T, C); state (1 + S, C): row 0 the previous token, rows 1.. the WKV state
 * ((S, C) read as (H, S, S) by a row-major reshape); v_first (T, C) (read when
 * layer_id > 0, written when layer_id == 0).  Outputs out (T, C) and the new
 * state (1 + S, C).  Weights as the reference module: mixes x_r..x_g (C);
 * Linear weights (out, in); Tmm weights (in, out). */
void or_time_mixing(const or_tm_weights *P, const float *x, int32_t T, int32_t C, int32_t H,
                    const float *state, float *v_first, int32_t length, const uint8_t *new_starts,
                    int32_t layer_id, float *out, float *state_out) {
    const int32_t S = C / H;
    const int64_t TC = (int64_t)T * C;
    float *mix[6];
    for (int m = 0; m < 6; ++m) mix[m] = (float *)malloc(sizeof(float) * (size_t)TC + 4);
    const float *mv[6] = {P->x_r, P->x_w, P->x_k, P->x_v, P->x_a, P->x_g};
    for (int32_t t = 0; t < T; ++t)
        for (int32_t c = 0; c < C; ++c) {
            float prev = t == 0 ? state[c] : x[(int64_t)(t - 1) * C + c];
            if (new_starts && new_starts[t]) prev = 0.0f;
            const float sx = prev - x[(int64_t)t * C + c];
            for (int m = 0; m < 6; ++m) mix[m][(int64_t)t * C + c] = x[(int64_t)t * C + c] + sx * mv[m][c];
        }
    float *r = (float *)malloc(sizeof(float) * (size_t)TC + 4);
    float *w = (float *)malloc(sizeof(float) * (size_t)TC + 4);
    float *k = (float *)malloc(sizeof(float) * (size_t)TC + 4);
    float *v = (float *)malloc(sizeof(float) * (size_t)TC + 4);
    float *a = (float *)malloc(sizeof(float) * (size_t)TC + 4);
    float *g = (float *)malloc(sizeof(float) * (size_t)TC + 4);
    float *tmp = (float *)malloc(sizeof(float) * (size_t)TC + 4);
    int32_t D = P->d_w;
    if (P->d_v > D) D = P->d_v;
    if (P->d_a > D) D = P->d_a;
    if (P->d_g > D) D = P->d_g;
    float *low = (float *)malloc(sizeof(float) * (size_t)T * D + 4);
    or_matmul_abt(mix[0], T, C, P->receptance, C, r);
    /* w = -softplus(-(w0 + w2(tanh(w1 xw)))) - 0.5 */
    matmul_ab_f32(mix[1], T, C, P->w1, P->d_w, low);
    for (int64_t e = 0; e < (int64_t)T * P->d_w; ++e) low[e] = tanhf(low[e]);
    matmul_ab_f32(low, T, P->d_w, P->w2, C, tmp);
    for (int64_t e = 0; e < TC; ++e) w[e] = -softplusf_(-(P->w0[e % C] + tmp[e])) - 0.5f;
    or_matmul_abt(mix[2], T, C, P->key, C, k);
    or_matmul_abt(mix[3], T, C, P->value, C, v);
    if (layer_id == 0) {
        memcpy(v_first, v, sizeof(float) * (size_t)TC);
    } else {
        matmul_ab_f32(mix[3], T, C, P->v1, P->d_v, low);
        for (int64_t e = 0; e < (int64_t)T * P->d_v; ++e) low[e] = tanhf(low[e]);
        matmul_ab_f32(low, T, P->d_v, P->v2, C, tmp);
        for (int64_t e = 0; e < TC; ++e)
            v[e] = v[e] + (v_first[e] - v[e]) * sigmoidf_(P->v0[e % C] + tmp[e]);
    }
    matmul_ab_f32(mix[4], T, C, P->a1, P->d_a, low);
    for (int64_t e = 0; e < (int64_t)T * P->d_a; ++e) low[e] = tanhf(low[e]);
    matmul_ab_f32(low, T, P->d_a, P->a2, C, tmp);
    for (int64_t e = 0; e < TC; ++e) a[e] = sigmoidf_(P->a0[e % C] + tmp[e]);
    matmul_ab_f32(mix[5], T, C, P->g1, P->d_g, low);
    for (int64_t e = 0; e < (int64_t)T * P->d_g; ++e) low[e] = sigmoidf_(low[e]);
    matmul_ab_f32(low, T, P->d_g, P->g2, C, g);
    /* kk = normalize_per_head(k * k_k); k = k * (k_a * (a - 1) + 1); a_i = -kk, b_i = kk * a */
    float *ai = (float *)malloc(sizeof(float) * (size_t)TC + 4);
    float *bi = (float *)malloc(sizeof(float) * (size_t)TC + 4);
    for (int32_t t = 0; t < T; ++t)
        for (int32_t h = 0; h < H; ++h) {
            const int64_t o = (int64_t)t * C + (int64_t)h * S;
            float ss = 0.0f;
            for (int32_t s = 0; s < S; ++s) {
                const float kk2 = k[o + s] * P->k_k[h * S + s];
                ss = ss + kk2 * kk2;
            }
            float nrm = sqrtf(ss);
            nrm = nrm < 1e-12f ? 1e-12f : nrm;
            for (int32_t s = 0; s < S; ++s) {
                const int32_t c = h * S + s;
                const float kk = (k[o + s] * P->k_k[c]) / nrm;
                ai[o + s] = -kk;
                bi[o + s] = kk * a[o + s];
                k[o + s] = k[o + s] * (P->k_a[c] * (a[o + s] - 1.0f) + 1.0f);
            }
        }
    /* the recurrence on state rows 1.. (a row-major (S, C) == (H, S, S) block) */
    float *wkv = (float *)malloc(sizeof(float) * (size_t)TC + 4);
    memcpy(state_out, state, sizeof(float) * (size_t)(1 + S) * C);
    memcpy(state_out, x + (int64_t)(length - 1) * C, sizeof(float) * (size_t)C);
    or_rwkv7_inner_loop(r, w, k, v, ai, bi, state + C, T, H, S, length, new_starts, wkv,
                        state_out + C);
    /* group norm per head (eps 64e-5), + readout (sum_s r k r_k) v, * g, output */
    or_group_norm(wkv, T, C, 1, H, P->ln_w, P->ln_b, 64e-5f, tmp);
    for (int32_t t = 0; t < T; ++t)
        for (int32_t h = 0; h < H; ++h) {
            const int64_t o = (int64_t)t * C + (int64_t)h * S;
            float sum = 0.0f;
            for (int32_t s = 0; s < S; ++s) sum = sum + r[o + s] * k[o + s] * P->r_k[h * S + s];
            for (int32_t s = 0; s < S; ++s) tmp[o + s] = (tmp[o + s] + sum * v[o + s]) * g[o + s];
        }
    or_matmul_abt(tmp, T, C, P->output, C, out);
    free(wkv);
    free(bi);
    free(ai);
    free(low);
    free(tmp);
    free(g);
    free(a);
    free(v);
    free(k);
    free(w);
    free(r);
    for (int m = 0; m < 6; ++m) free(mix[m]);
}

/* rwkv7.py:189-253: x = ln0(emb[tokens]); per block x += att(ln1(x)), x += ffn(ln2(x))
 * with v_first carried from block 0; logits = ln_out(x) head^T.  LayerNorm eps 1e-5
 * (rwkv7.py:32). */
void or_rwkv_lm_forward(const or_rwkv_lm *P, const int32_t *tokens, int32_t T, float *state,
                        float *logits) {
    const int32_t C = P->C, H = P->H, S = C / H;
    const int64_t TC = (int64_t)T * C, SR = (int64_t)(2 + S) * C;
    float *x = (float *)malloc(sizeof(float) * (size_t)TC + 4);
    float *h = (float *)malloc(sizeof(float) * (size_t)TC + 4);
    float *d = (float *)malloc(sizeof(float) * (size_t)TC + 4);
    float *vf = (float *)calloc((size_t)TC + 1, sizeof(float));
    float *st = (float *)malloc(sizeof(float) * (size_t)(1 + S) * C + 4);
    for (int32_t t = 0; t < T; ++t)
        memcpy(x + (int64_t)t * C, P->emb + (int64_t)tokens[t] * C, sizeof(float) * (size_t)C);
    or_layer_norm(x, T, C, P->ln0_w, P->ln0_b, 1e-5f, h);
    memcpy(x, h, sizeof(float) * (size_t)TC);
    for (int32_t l = 0; l < P->n_layer; ++l) {
        const or_rwkv_block *B = &P->blocks[l];
        float *sl = state + (int64_t)l * SR;
        or_layer_norm(x, T, C, B->ln1_w, B->ln1_b, 1e-5f, h);
        or_time_mixing(&B->tm, h, T, C, H, sl + C, vf, T, NULL, l, d, st);
        memcpy(sl + C, st, sizeof(float) * (size_t)(1 + S) * C);
        for (int64_t e = 0; e < TC; ++e) x[e] = x[e] + d[e];
        or_layer_norm(x, T, C, B->ln2_w, B->ln2_b, 1e-5f, h);
        or_channel_mixing(h, T, C, sl, B->ffn_x_k, B->ffn_key, P->F, B->ffn_value, T, NULL, d, st);
        memcpy(sl, st, sizeof(float) * (size_t)C);
        for (int64_t e = 0; e < TC; ++e) x[e] = x[e] + d[e];
    }
    or_layer_norm(x, T, C, P->ln_out_w, P->ln_out_b, 1e-5f, h);
    or_matmul_abt(h, T, C, P->head, P->V, logits);
    free(st);
    free(vf);
    free(d);
    free(h);
    free(x);
}
