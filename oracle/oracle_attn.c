/* oracle_attn.c -- CPU restatement of the spiking self-attention transformer
 * (C4) for one population member.  Test infrastructure only.
 *
 * Follows src/hyperscalees/models/snn_self_attention_heads.py (the JAX model
 * with LIF-encoded Q/K/V, multi-head row_softmax_lif attention, the LIF-gated
 * feed-forward and the pooled readout) with the LIF step of
 * src/hyperscalees/models/snn_attention.py:41-61 and row_softmax_lif of
 * src/hyperscalees/models/snn_self_attention.py:45-80.  Every operation is a
 * single f32 IEEE operation in the order the reference writes it
 * (-ffp-contract=off); reductions are sequential in index order.
 * The member's parameters come in materialised (W + A_m B_m^T for the MM
 * leaves, param + noise for the Parameter leaves). */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* jax.nn.softplus(x) = logaddexp(x, 0) = max(x, 0) + log1p(exp(-|x|)). */
float or_sa_softplus(float x) {
    return fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x)));
}

/* snn_attention.py:41-49: v + (dt/tau_m) * (-v + current); spike = v >= v_th;
 * hard reset v * (1 - spike).  dt = 1. */
static float lif_update(float v, float cur, float leak, float vth, float *spike) {
    float vn = v + leak * (-v + cur);
    float s = vn >= vth ? 1.0f : 0.0f;
    *spike = s;
    return vn * (1.0f - s);
}

/* snn_self_attention_heads.py:33-40 (_rate) for the three encoders and the
 * encoder sum (:168-175): X = (rate(cq) + rate(ck) + rate(cv)) / 3 + pos.
 * c* are time-major (T, R, d) projection currents of one member. */
void or_sa_encode(const float *cq, const float *ck, const float *cv, int32_t T, int32_t R,
                  int32_t d, float th_q, float th_k, float th_v, float tau_m, const float *pos,
                  float *X) {
    const float leak = 1.0f / tau_m;
    const float *cs[3] = {cq, ck, cv};
    const float th[3] = {th_q, th_k, th_v};
    for (int64_t e = 0; e < (int64_t)R * d; ++e) {
        float rate[3];
        for (int q = 0; q < 3; ++q) {
            float v = 0.0f, cnt = 0.0f, s;
            for (int32_t t = 0; t < T; ++t) {
                v = lif_update(v, cs[q][(int64_t)t * R * d + e], leak, th[q], &s);
                cnt = cnt + s;
            }
            rate[q] = cnt / (float)T; /* jnp.mean over T */
        }
        X[e] = ((rate[0] + rate[1]) + rate[2]) / 3.0f + pos[e];
    }
}

/* snn_self_attention.py:45-80: p_j = count_j / (sum count + 1e-6) after
 * n_iter LIF steps of the key neurons on the row-normalised currents
 * h_j / (max |h| + 1e-6) minus the global inhibition g_inh * sum(count). */
void or_sa_row_softmax_lif(const float *h, int32_t n, float vth, float g_inh, float tau_m,
                           int32_t n_iter, float *p) {
    float mx = 0.0f;
    for (int32_t j = 0; j < n; ++j) mx = fmaxf(mx, fabsf(h[j]));
    const float den = mx + 1e-6f, leak = 1.0f / tau_m;
    float *hn = (float *)malloc(sizeof(float) * (size_t)n + 4);
    float *u = (float *)calloc((size_t)n + 1, sizeof(float));
    float *cnt = (float *)calloc((size_t)n + 1, sizeof(float));
    for (int32_t j = 0; j < n; ++j) hn[j] = h[j] / den;
    for (int32_t it = 0; it < n_iter; ++it) {
        float G = 0.0f;
        for (int32_t j = 0; j < n; ++j) G = G + cnt[j];
        const float inh = g_inh * G;
        for (int32_t j = 0; j < n; ++j) {
            float s;
            u[j] = lif_update(u[j], hn[j] - inh, leak, vth, &s);
            cnt[j] = cnt[j] + s;
        }
    }
    float tot = 0.0f;
    for (int32_t j = 0; j < n; ++j) tot = tot + cnt[j];
    for (int32_t j = 0; j < n; ++j) p[j] = cnt[j] / (tot + 1e-6f);
    free(hn);
    free(u);
    free(cnt);
}

/* One head of multihead_attention_once (snn_self_attention_heads.py:54-70):
 * h_i = beta * (q_i . k_j) over keys j, p_i = row_softmax_lif(h_i), out_i =
 * p_i @ V.  q, k, v, out are (R, hd) rows with row stride ld. */
void or_sa_attention_head(const float *q, const float *k, const float *v, int32_t R, int32_t hd,
                          int32_t ld, float beta, float vth, float g_inh, float tau_m,
                          int32_t n_iter, float *out) {
    float *h = (float *)malloc(sizeof(float) * (size_t)R + 4);
    float *p = (float *)malloc(sizeof(float) * (size_t)R + 4);
    for (int32_t i = 0; i < R; ++i) {
        for (int32_t j = 0; j < R; ++j) {
            float s = 0.0f;
            for (int32_t c = 0; c < hd; ++c) s = s + q[(int64_t)i * ld + c] * k[(int64_t)j * ld + c];
            h[j] = beta * s;
        }
        or_sa_row_softmax_lif(h, R, vth, g_inh, tau_m, n_iter, p);
        for (int32_t c = 0; c < hd; ++c) {
            float s = 0.0f;
            for (int32_t j = 0; j < R; ++j) s = s + p[j] * v[(int64_t)j * ld + c];
            out[(int64_t)i * ld + c] = s;
        }
    }
    free(h);
    free(p);
}

/* ffn_once's lif_single (snn_self_attention_heads.py:79-83), per row:
 * spike = c / max(max |c|, 1e-6) >= vth. */
void or_sa_ffn_spike(const float *c, int32_t R, int32_t d, float vth, float *act) {
    for (int32_t i = 0; i < R; ++i) {
        const float *row = c + (int64_t)i * d;
        float mx = 0.0f;
        for (int32_t j = 0; j < d; ++j) mx = fmaxf(mx, fabsf(row[j]));
        const float den = fmaxf(mx, 1e-6f);
        for (int32_t j = 0; j < d; ++j) act[(int64_t)i * d + j] = (row[j] / den >= vth) ? 1.0f : 0.0f;
    }
}

/* y (rows, out) = x (rows, in) @ W^T, f32 accumulation in ascending k. */
static void mm_t(const float *x, int32_t rows, int32_t in, const float *W, int32_t out, float *y,
                 int32_t ldy, int32_t y_off) {
    for (int32_t i = 0; i < rows; ++i)
        for (int32_t o = 0; o < out; ++o) {
            float s = 0.0f;
            for (int32_t k = 0; k < in; ++k) s = s + x[(int64_t)i * in + k] * W[(int64_t)o * in + k];
            y[(int64_t)i * ldy + y_off + o] = s;
        }
}

/* SNNSelfAttentionHeadsModel._forward (snn_self_attention_heads.py:161-189)
 * for one member: x (T, R, tin) input spikes -> logits (classes). */
void or_sa_forward_member(const or_sa_cfg *cfg, const or_sa_params *P, const float *x,
                          float *logits) {
    const int32_t T = cfg->T, R = cfg->ntok, tin = cfg->tin, d = cfg->d_model, H = cfg->heads;
    const int32_t hd = d / H, nb = cfg->blocks, C = cfg->classes;
    const size_t rd = (size_t)R * d;
    float *cq = (float *)malloc(sizeof(float) * (size_t)T * rd + 4);
    float *ck = (float *)malloc(sizeof(float) * (size_t)T * rd + 4);
    float *cv = (float *)malloc(sizeof(float) * (size_t)T * rd + 4);
    for (int32_t t = 0; t < T; ++t) {
        const float *xt = x + (int64_t)t * R * tin;
        mm_t(xt, R, tin, P->in_q, d, cq + (int64_t)t * rd, d, 0);
        mm_t(xt, R, tin, P->in_k, d, ck + (int64_t)t * rd, d, 0);
        mm_t(xt, R, tin, P->in_v, d, cv + (int64_t)t * rd, d, 0);
    }
    float *X = (float *)malloc(sizeof(float) * rd + 4);
    or_sa_encode(cq, ck, cv, T, R, d, or_sa_softplus(P->q_th), or_sa_softplus(P->k_th),
                 or_sa_softplus(P->v_th), cfg->tau_m, P->pos, X);
    const float beta = or_sa_softplus(P->beta);
    const float vth_attn = or_sa_softplus(P->attn_th);
    float *Q = (float *)malloc(sizeof(float) * rd + 4);
    float *K = (float *)malloc(sizeof(float) * rd + 4);
    float *V = (float *)malloc(sizeof(float) * rd + 4);
    float *O = (float *)malloc(sizeof(float) * rd + 4);
    float *D = (float *)malloc(sizeof(float) * rd + 4);
    for (int32_t b = 0; b < nb; ++b) {
        const or_sa_block *B = &P->blocks[b];
        for (int32_t h = 0; h < H; ++h) {
            mm_t(X, R, d, B->q[h], hd, Q, d, h * hd);
            mm_t(X, R, d, B->k[h], hd, K, d, h * hd);
            mm_t(X, R, d, B->v[h], hd, V, d, h * hd);
            or_sa_attention_head(Q + h * hd, K + h * hd, V + h * hd, R, hd, d, beta, vth_attn,
                                 cfg->g_inh, cfg->tau_m, cfg->n_iter, O + h * hd);
        }
        mm_t(O, R, d, B->o, d, D, d, 0);
        for (size_t e = 0; e < rd; ++e) X[e] = X[e] + D[e];
        mm_t(X, R, d, B->ff1, d, D, d, 0);
        or_sa_ffn_spike(D, R, d, or_sa_softplus(B->ff_th), O);
        mm_t(O, R, d, B->ff2, d, D, d, 0);
        for (size_t e = 0; e < rd; ++e) X[e] = X[e] + D[e];
    }
    float *pooled = (float *)malloc(sizeof(float) * (size_t)d + 4);
    for (int32_t c = 0; c < d; ++c) {
        float s = 0.0f;
        for (int32_t i = 0; i < R; ++i) s = s + X[(int64_t)i * d + c];
        pooled[c] = s / (float)R; /* jnp.mean(X, axis=0) */
    }
    mm_t(pooled, 1, d, P->out, C, logits, C, 0);
    for (int32_t c = 0; c < C; ++c) logits[c] = logits[c] * P->out_gain;
    free(cq);
    free(ck);
    free(cv);
    free(X);
    free(Q);
    free(K);
    free(V);
    free(O);
    free(D);
    free(pooled);
}
