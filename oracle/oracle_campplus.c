/*
 * oracle_campplus.c - CPU restatement of the reference CAM++ encoder
 * (src/encoder_campplus.cpp).  TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Per clip, channel-major like the reference's dense backbone: the FCM front
 * end is NCHW [C][H=freq][W=time], the D-TDNN backbone [C][T'].  Arithmetic in
 * f32; time means are accumulated in double.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* Fixed CAM++ dense topology (src/encoder_campplus.cpp:197-198). */
static const int kLayers[3] = {12, 24, 16};
static const int kDil[3] = {1, 2, 2};
static const int kSeg = 100;   /* context segment length (src/encoder_campplus.cpp:170-182) */

static void bn_relu(const float* x, int C, int T, const orc_bn* bn, float eps, float* y) {
    /* src/encoder_campplus.cpp:110-134: scale = g/sqrt(var+eps), shift = b - scale*mu, then ReLU */
    for (int c = 0; c < C; ++c) {
        const float inv = bn->gamma[c] / sqrtf(bn->var[c] + eps);
        const float sh = bn->beta[c] - inv * bn->mean[c];
        const float* r = x + (size_t)c * T;
        float* o = y + (size_t)c * T;
        for (int t = 0; t < T; ++t) {
            const float v = r[t] * inv + sh;
            o[t] = v > 0.0f ? v : 0.0f;
        }
    }
}

/* 1-D conv over [ic][T] (H = 1) with zero padding, stride and dilation. */
static void conv1d(const orc_conv* c, const float* x, int T, int stride, int pad, int dil, int relu, float* y) {
    orc_conv2d_f32_g(x, c->ic, 1, T, c->w, c->oc, 1, c->kw, 1, stride, 0, pad, 1, dil, c->b, NULL, relu, y);
}

/* FCM BasicResBlock (src/encoder_campplus.cpp:136-146): conv1 (3x3, freq
 * stride) -> ReLU -> conv2 (3x3) -> + shortcut (1x1 freq-stride conv when
 * stride != 1) -> ReLU. */
static float* fcm_block(const orc_campplus* n, int* ci, const float* x, int C, int* H, int W, int stride) {
    const orc_conv* c1 = &n->conv[(*ci)++];
    const orc_conv* c2 = &n->conv[(*ci)++];
    const int Ho = (*H + 2 - 3) / stride + 1;
    float* h = malloc(sizeof(float) * (size_t)c1->oc * Ho * W);
    orc_conv2d_f32_g(x, C, *H, W, c1->w, c1->oc, 3, 3, stride, 1, 1, 1, 1, 1, c1->b, NULL, 1, h);
    float* res = NULL;
    const float* r = x;
    if (stride != 1) {
        const orc_conv* sc = &n->conv[(*ci)++];
        res = malloc(sizeof(float) * (size_t)sc->oc * Ho * W);
        orc_conv2d_f32_g(x, C, *H, W, sc->w, sc->oc, 1, 1, stride, 1, 0, 0, 1, 1, sc->b, NULL, 0, res);
        r = res;
    }
    float* y = malloc(sizeof(float) * (size_t)c2->oc * Ho * W);
    orc_conv2d_f32_g(h, c1->oc, Ho, W, c2->w, c2->oc, 3, 3, 1, 1, 1, 1, 1, 1, c2->b, r, 1, y);
    free(h);
    free(res);
    *H = Ho;
    return y;
}

int orc_campplus_forward(const orc_campplus* n, const float* feats, int T, float* emb, orc_campplus_caps* caps) {
    int ci = 0, bi = 0;
    const float eps = n->bn_eps;
    /* FCM: stem 3x3 -> ReLU, BasicResBlocks (freq strides 2,1,2,1), final 3x3 freq-s2 -> ReLU */
    int H = n->n_mels, C = n->conv[0].oc;
    float* x = malloc(sizeof(float) * (size_t)C * H * T);
    orc_conv2d_f32_g(feats, 1, H, T, n->conv[0].w, C, 3, 3, 1, 1, 1, 1, 1, 1, n->conv[0].b, NULL, 1, x);
    ci = 1;
    const int strides[4] = {2, 1, 2, 1};
    for (int i = 0; i < 4; ++i) {
        float* y = fcm_block(n, &ci, x, C, &H, T, strides[i]);
        free(x);
        x = y;
        C = n->conv[ci - 1].oc;
    }
    {
        const orc_conv* c2 = &n->conv[ci++];
        const int Ho = (H + 2 - 3) / 2 + 1;
        float* y = malloc(sizeof(float) * (size_t)c2->oc * Ho * T);
        orc_conv2d_f32_g(x, C, H, T, c2->w, c2->oc, 3, 3, 2, 1, 1, 1, 1, 1, c2->b, NULL, 1, y);
        free(x);
        x = y;
        C = c2->oc;
        H = Ho;
    }
    /* [C][H][T] is already the [C*H][T] TDNN input (channel c*H + h). */
    const int Cf = C * H;
    if (caps && caps->fcm) memcpy(caps->fcm, x, sizeof(float) * (size_t)Cf * T);

    /* TDNN: Conv1d(k=5, stride 2, pad 2) -> ReLU (src/encoder_campplus.cpp:236-239) */
    const orc_conv* td = &n->conv[ci++];
    const int Tp = (T - 1) / 2 + 1;
    int Ccur = td->oc;
    /* widest dense state over the three blocks */
    int cmax = Ccur, cw = Ccur;
    {
        int cj = ci;
        for (int b = 0; b < 3; ++b) {
            for (int l = 0; l < kLayers[b]; ++l) {
                cw += n->conv[cj + 1].oc;   /* linear_local output = growth */
                cj += 4;
            }
            if (cw > cmax) cmax = cw;
            cw = n->conv[cj].oc;            /* transit */
            cj += 1;
        }
    }
    float* h = malloc(sizeof(float) * (size_t)cmax * Tp);
    conv1d(td, x, T, 2, 2, 1, 1, h);
    free(x);
    if (caps && caps->tdnn) memcpy(caps->tdnn, h, sizeof(float) * (size_t)Ccur * Tp);

    const int nseg = (Tp + kSeg - 1) / kSeg;
    float* a = malloc(sizeof(float) * (size_t)cmax * Tp);
    float* tmp = malloc(sizeof(float) * (size_t)cmax * Tp);
    for (int b = 0; b < 3; ++b) {
        const int dil = kDil[b];
        for (int l = 0; l < kLayers[b]; ++l) {
            const orc_conv* l1 = &n->conv[ci++];
            const orc_conv* ll = &n->conv[ci++];
            const orc_conv* c1 = &n->conv[ci++];
            const orc_conv* c2 = &n->conv[ci++];
            /* nonlinear1: BN -> ReLU; linear1 (+folded BN) -> ReLU */
            bn_relu(h, Ccur, Tp, &n->bn[bi++], eps, a);
            float* cc = tmp;
            conv1d(l1, a, Tp, 1, 0, 1, 1, cc);
            const int bc = l1->oc;
            /* linear_local: k=3, dilation dil, same zero padding */
            float* y = a;   /* a is free again */
            conv1d(ll, cc, Tp, 1, dil, dil, 0, y);
            /* context = mean over T' + 100-frame segment average (count_include_pad) */
            float* ctx = malloc(sizeof(float) * (size_t)bc * nseg);
            for (int c = 0; c < bc; ++c) {
                const float* r = cc + (size_t)c * Tp;
                double s = 0.0;
                for (int t = 0; t < Tp; ++t) s += r[t];
                const float m = (float)(s / Tp);
                for (int sg = 0; sg < nseg; ++sg) {
                    double ss = 0.0;
                    const int t1 = (sg + 1) * kSeg < Tp ? (sg + 1) * kSeg : Tp;
                    for (int t = sg * kSeg; t < t1; ++t) ss += r[t];
                    ctx[(size_t)c * nseg + sg] = m + (float)(ss / kSeg);
                }
            }
            /* linear1 -> ReLU -> linear2 -> sigmoid, per segment (the context is
             * constant over a segment's frames) */
            float* hc = malloc(sizeof(float) * (size_t)c1->oc * nseg);
            conv1d(c1, ctx, nseg, 1, 0, 1, 1, hc);
            float* m = malloc(sizeof(float) * (size_t)c2->oc * nseg);
            conv1d(c2, hc, nseg, 1, 0, 1, 0, m);
            for (size_t i = 0; i < (size_t)c2->oc * nseg; ++i) m[i] = 1.0f / (1.0f + expf(-m[i]));
            /* out = y * m appended to the dense state */
            const int g = ll->oc;
            for (int c = 0; c < g; ++c) {
                float* o = h + (size_t)(Ccur + c) * Tp;
                const float* yr = y + (size_t)c * Tp;
                for (int t = 0; t < Tp; ++t) o[t] = yr[t] * m[(size_t)c * nseg + t / kSeg];
            }
            Ccur += g;
            free(ctx);
            free(hc);
            free(m);
        }
        /* transit: BN -> ReLU -> 1x1 (c -> c/2); the last adds the out ReLU */
        const orc_conv* tr = &n->conv[ci++];
        bn_relu(h, Ccur, Tp, &n->bn[bi++], eps, a);
        conv1d(tr, a, Tp, 1, 0, 1, b == 2, h);
        Ccur = tr->oc;
        if (caps && caps->block[b]) memcpy(caps->block[b], h, sizeof(float) * (size_t)Ccur * Tp);
    }
    free(a);
    free(tmp);

    /* stats pooling: mean + unbiased std, no eps (src/encoder_campplus.cpp:284-296) */
    float* pooled = malloc(sizeof(float) * 2 * (size_t)Ccur);
    orc_tstp(h, Ccur, 1, Tp, 0.0f, pooled);
    free(h);
    if (caps && caps->pooled) memcpy(caps->pooled, pooled, sizeof(float) * 2 * (size_t)Ccur);

    /* dense 1x1 (2C -> emb) then the affine-free BN (src/encoder_campplus.cpp:299-306) */
    const orc_conv* dn = &n->conv[ci++];
    orc_linear(pooled, 2 * Ccur, dn->w, dn->b, NULL, dn->oc, emb);
    free(pooled);
    for (int i = 0; i < dn->oc; ++i) {
        const float inv = 1.0f / sqrtf(n->emb_var[i] + eps);
        const float sh = 0.0f - inv * n->emb_mean[i];
        emb[i] = emb[i] * inv + sh;
    }
    if (caps && caps->pre_norm) memcpy(caps->pre_norm, emb, sizeof(float) * (size_t)dn->oc);
    if (n->l2_normalize) orc_l2norm(emb, dn->oc);
    return ci == n->n_conv && bi == n->n_bn ? 0 : 1;
}
