/*
 * oracle_ecapa.c - CPU restatement of the reference ECAPA-TDNN encoder
 * (src/encoder.cpp).  TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Layout per clip is channel-major [C][T] (the reference's ggml [T, C] with
 * time fastest).  Arithmetic in f32 like the reference's ggml graph; means and
 * the softmax normaliser are accumulated in double.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

static const float kBnEps = 1e-5f;    /* src/encoder.cpp:13 */
static const float kAspEps = 1e-12f;  /* src/encoder.cpp:19 */

void orc_conv1d_same(const float* x, int T, const orc_conv1d* c, int dilation, float* y) {
    const int pad = ((c->k - 1) / 2) * dilation, Tp = T + 2 * pad;
    float* xp = malloc(sizeof(float) * (size_t)c->ic * Tp);
    for (int ic = 0; ic < c->ic; ++ic) {
        const float* xr = x + (size_t)ic * T;
        float* pr = xp + (size_t)ic * Tp;
        for (int j = 0; j < Tp; ++j) {
            int t;
            if (j < pad) t = pad - j;                    /* left reflect, no edge repeat */
            else if (j < pad + T) t = j - pad;
            else t = (T - 2) - (j - pad - T);            /* right reflect */
            if (t < 0) t = 0;                            /* only reachable when T < pad + 1, */
                                                         /* a length the library refuses */
            if (t > T - 1) t = T - 1;
            pr[j] = xr[t];
        }
    }
    for (int oc = 0; oc < c->oc; ++oc) {
        float* yr = y + (size_t)oc * T;
        for (int t = 0; t < T; ++t) yr[t] = 0.0f;
        for (int ic = 0; ic < c->ic; ++ic)
            for (int k = 0; k < c->k; ++k) {
                const float wv = c->w[((size_t)oc * c->ic + ic) * c->k + k];
                const float* pr = xp + (size_t)ic * Tp + k * dilation;
                for (int t = 0; t < T; ++t) yr[t] += wv * pr[t];
            }
        const float bv = c->b ? c->b[oc] : 0.0f;
        for (int t = 0; t < T; ++t) yr[t] += bv;
    }
    free(xp);
}

void orc_bn_apply(float* x, int T, const orc_bn* bn) {
    for (int c = 0; c < bn->c; ++c) {
        const float inv = bn->gamma[c] / sqrtf(bn->var[c] + kBnEps);
        const float shift = bn->beta[c] - inv * bn->mean[c];
        float* r = x + (size_t)c * T;
        for (int t = 0; t < T; ++t) r[t] = r[t] * inv + shift;
    }
}

static void relu_inplace(float* x, size_t n) {
    for (size_t i = 0; i < n; ++i)
        if (x[i] < 0.0f) x[i] = 0.0f;
}

/* TDNNBlock: Conv1d -> ReLU -> BN (src/encoder.cpp:157-167). */
static void tdnn_block(const float* x, int T, const orc_conv1d* c, const orc_bn* bn, int dil, float* y) {
    orc_conv1d_same(x, T, c, dil, y);
    relu_inplace(y, (size_t)c->oc * T);
    orc_bn_apply(y, T, bn);
}

static float mean_row(const float* r, int T) {
    double s = 0.0;
    for (int t = 0; t < T; ++t) s += r[t];
    return (float)(s / T);
}

void orc_ecapa_asp(const orc_ecapa* net, const float* x, int T, float* pooled) {
    const int C = net->mfa_ch;
    const int A = net->asp_tdnn.oc;
    float* ctx = malloc(sizeof(float) * (size_t)3 * C * T);
    memcpy(ctx, x, sizeof(float) * (size_t)C * T);
    for (int c = 0; c < C; ++c) {                     /* global mean / std, clamp not add */
        const float* r = x + (size_t)c * T;
        const float m = mean_row(r, T);
        double s2 = 0.0;
        for (int t = 0; t < T; ++t) { const float d = r[t] - m; s2 += (double)(d * d); }
        float v = (float)(s2 / T);
        if (v < kAspEps) v = kAspEps;
        const float sd = sqrtf(v);
        for (int t = 0; t < T; ++t) {
            ctx[(size_t)(C + c) * T + t] = m;
            ctx[(size_t)(2 * C + c) * T + t] = sd;
        }
    }
    float* a1 = malloc(sizeof(float) * (size_t)A * T);
    tdnn_block(ctx, T, &net->asp_tdnn, &net->bn_asp, 1, a1);
    for (size_t i = 0; i < (size_t)A * T; ++i) a1[i] = tanhf(a1[i]);
    float* lg = malloc(sizeof(float) * (size_t)C * T);
    orc_conv1d_same(a1, T, &net->asp_conv, 1, lg);
    for (int c = 0; c < C; ++c) {
        float* l = lg + (size_t)c * T;
        const float* r = x + (size_t)c * T;
        float mx = l[0];
        for (int t = 1; t < T; ++t) if (l[t] > mx) mx = l[t];
        double z = 0.0;
        for (int t = 0; t < T; ++t) { l[t] = expf(l[t] - mx); z += l[t]; }
        for (int t = 0; t < T; ++t) l[t] = (float)(l[t] / z);       /* softmax over time */
        double mu = 0.0;
        for (int t = 0; t < T; ++t) mu += (double)l[t] * r[t];
        const float muf = (float)mu;
        double var = 0.0;
        for (int t = 0; t < T; ++t) { const float d = r[t] - muf; var += (double)l[t] * (d * d); }
        float v = (float)var;
        if (v < kAspEps) v = kAspEps;
        pooled[c] = muf;
        pooled[C + c] = sqrtf(v);
    }
    free(ctx); free(a1); free(lg);
}

int orc_ecapa_forward(const orc_ecapa* net, const float* feats, int T, float* emb, orc_ecapa_caps* caps) {
    const int C = net->channels, G = C / net->scale, R = net->n_res;
    float* h = malloc(sizeof(float) * (size_t)C * T);
    tdnn_block(feats, T, &net->block0, &net->bn0, 1, h);             /* block0 */
    if (caps && caps->block[0]) memcpy(caps->block[0], h, sizeof(float) * (size_t)C * T);
    float* cat = malloc(sizeof(float) * (size_t)R * C * T);
    float* t1 = malloc(sizeof(float) * (size_t)C * T);
    float* r2 = malloc(sizeof(float) * (size_t)C * T);
    float* t2 = malloc(sizeof(float) * (size_t)C * T);
    float* in = malloc(sizeof(float) * (size_t)G * T);
    float* se = malloc(sizeof(float) * (size_t)C);
    float* sh = malloc(sizeof(float) * (size_t)C);
    const float* x = h;
    for (int i = 0; i < R; ++i) {                                     /* SE-Res2Net blocks */
        const int dil = i + 2;                                        /* block index + 1 */
        tdnn_block(x, T, &net->tdnn1[i], &net->bn_t1[i], 1, t1);
        memcpy(r2, t1, sizeof(float) * (size_t)G * T);                /* group 0 passthrough */
        for (int j = 1; j < net->scale; ++j) {
            const float* xj = t1 + (size_t)j * G * T;
            if (j == 1) memcpy(in, xj, sizeof(float) * (size_t)G * T);
            else {
                const float* yp = r2 + (size_t)(j - 1) * G * T;
                for (size_t q = 0; q < (size_t)G * T; ++q) in[q] = xj[q] + yp[q];
            }
            tdnn_block(in, T, &net->res[i][j - 1], &net->bn_res[i][j - 1], dil, r2 + (size_t)j * G * T);
        }
        tdnn_block(r2, T, &net->tdnn2[i], &net->bn_t2[i], 1, t2);
        for (int c = 0; c < C; ++c) se[c] = mean_row(t2 + (size_t)c * T, T);   /* SE */
        orc_conv1d_same(se, 1, &net->se1[i], 1, sh);
        relu_inplace(sh, (size_t)net->se1[i].oc);
        orc_conv1d_same(sh, 1, &net->se2[i], 1, se);
        float* out = cat + (size_t)i * C * T;
        for (int c = 0; c < C; ++c) {
            const float g = 1.0f / (1.0f + expf(-se[c]));
            for (int t = 0; t < T; ++t)
                out[(size_t)c * T + t] = t2[(size_t)c * T + t] * g + x[(size_t)c * T + t];
        }
        if (caps && caps->block[i + 1]) memcpy(caps->block[i + 1], out, sizeof(float) * (size_t)C * T);
        x = out;
    }
    const int M = net->mfa_ch;
    float* mfa = malloc(sizeof(float) * (size_t)M * T);
    tdnn_block(cat, T, &net->mfa, &net->bn_mfa, 1, mfa);                   /* MFA */
    if (caps && caps->mfa) memcpy(caps->mfa, mfa, sizeof(float) * (size_t)M * T);
    float* pooled = malloc(sizeof(float) * (size_t)2 * M);
    orc_ecapa_asp(net, mfa, T, pooled);
    if (caps && caps->pooled) memcpy(caps->pooled, pooled, sizeof(float) * (size_t)2 * M);
    orc_bn_apply(pooled, 1, &net->asp_bn);                                  /* asp_bn */
    orc_conv1d_same(pooled, 1, &net->fc, 1, emb);                           /* fc */
    if (caps && caps->pre_norm) memcpy(caps->pre_norm, emb, sizeof(float) * net->emb_dim);
    if (net->l2_normalize) orc_l2norm(emb, net->emb_dim);
    free(h); free(cat); free(t1); free(r2); free(t2); free(in); free(se); free(sh); free(mfa); free(pooled);
    return 0;
}
