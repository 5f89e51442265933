/*
 * oracle_eres2net.c - CPU restatement of the reference ERes2Net encoder
 * (src/encoder_eres2net.cpp).  TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Per clip, NCHW [C][H=freq][W=time] f32.  Every conv takes its stride from
 * the manifest and "same" zero padding (K-1)/2 (src/encoder_eres2net.cpp:36-54).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

typedef struct {
    const orc_eres2net* n;
    int idx;
} cursor;

typedef struct {
    float* d;
    int C, H, W;
} fmap;

static fmap fm_new(int C, int H, int W) {
    fmap m = {malloc(sizeof(float) * (size_t)C * H * W), C, H, W};
    return m;
}

static void hclamp(float* x, size_t n, float hi) {
    /* Hardtanh(0, hi) (src/encoder_eres2net.cpp:60-62) */
    for (size_t i = 0; i < n; ++i) x[i] = x[i] < 0.0f ? 0.0f : (x[i] > hi ? hi : x[i]);
}

/* next conv in manifest order: stride from the manifest, pad (K-1)/2 */
static fmap next_conv(cursor* cur, fmap x, const float* residual) {
    const orc_conv* c = &cur->n->conv[cur->idx];
    const int s = cur->n->stride[cur->idx];
    ++cur->idx;
    const int ph = (c->kh - 1) / 2, pw = (c->kw - 1) / 2;
    const int Ho = (x.H + 2 * ph - c->kh) / s + 1, Wo = (x.W + 2 * pw - c->kw) / s + 1;
    fmap y = fm_new(c->oc, Ho, Wo);
    orc_conv2d_f32_g(x.d, x.C, x.H, x.W, c->w, c->oc, c->kh, c->kw, s, s, ph, pw, 1, 1, c->b, residual, 0, y.d);
    return y;
}

static size_t fm_n(fmap m) { return (size_t)m.C * m.H * m.W; }

/* AFF: z = conv2(silu(conv1(cat(x, ds)))); out = (x + ds) + tanh(z) * (x - ds)
 * (src/encoder_eres2net.cpp:91-101) */
static fmap aff(cursor* cur, fmap x, fmap ds) {
    fmap cat = fm_new(x.C + ds.C, x.H, x.W);
    memcpy(cat.d, x.d, sizeof(float) * fm_n(x));
    memcpy(cat.d + fm_n(x), ds.d, sizeof(float) * fm_n(ds));
    fmap z = next_conv(cur, cat, NULL);
    free(cat.d);
    for (size_t i = 0; i < fm_n(z); ++i) z.d[i] = z.d[i] / (1.0f + expf(-z.d[i]));
    fmap z2 = next_conv(cur, z, NULL);
    free(z.d);
    for (size_t i = 0; i < fm_n(z2); ++i) {
        const float a = x.d[i], b = ds.d[i];
        z2.d[i] = (a + b) + tanhf(z2.d[i]) * (a - b);
    }
    return z2;
}

/* Res2Net block, expansion 2 (src/encoder_eres2net.cpp:111-137). */
static fmap block(cursor* cur, fmap x, int planes, int stride, int is_aff, int* in_planes) {
    const float hi = cur->n->relu_clamp;
    const int scale = cur->n->scale;
    fmap out = next_conv(cur, x, NULL);
    hclamp(out.d, fm_n(out), hi);
    const int width = out.C / scale;
    const size_t plane = (size_t)out.H * out.W;
    fmap acc = fm_new(out.C, out.H, out.W);
    fmap sp = {NULL, 0, 0, 0};
    for (int i = 0; i < scale; ++i) {
        fmap chunk = {out.d + (size_t)i * width * plane, width, out.H, out.W};
        fmap in;
        int own = 0;
        if (i == 0) {
            in = chunk;
        } else if (is_aff) {
            in = aff(cur, sp, chunk);
            own = 1;
        } else {
            in = fm_new(width, out.H, out.W);
            for (size_t k = 0; k < fm_n(in); ++k) in.d[k] = sp.d[k] + chunk.d[k];
            own = 1;
        }
        fmap cv = next_conv(cur, in, NULL);
        if (own) free(in.d);
        hclamp(cv.d, fm_n(cv), hi);
        memcpy(acc.d + (size_t)i * width * plane, cv.d, sizeof(float) * fm_n(cv));
        if (sp.d) free(sp.d);
        sp = cv;
    }
    free(sp.d);
    free(out.d);
    /* conv3 (1x1) + shortcut, then clamp.  The shortcut conv follows conv3 in
     * the manifest; the residual is added after conv3's bias. */
    const orc_conv* c3 = &cur->n->conv[cur->idx];
    const int s3 = cur->n->stride[cur->idx];
    ++cur->idx;
    fmap res = x;
    int own_res = 0;
    if (stride != 1 || *in_planes != 2 * planes) {
        res = next_conv(cur, x, NULL);
        own_res = 1;
    }
    fmap y = fm_new(c3->oc, acc.H, acc.W);
    orc_conv2d_f32_g(acc.d, acc.C, acc.H, acc.W, c3->w, c3->oc, c3->kh, c3->kw, s3, s3, 0, 0, 1, 1, c3->b, res.d, 0,
                     y.d);
    free(acc.d);
    if (own_res) free(res.d);
    hclamp(y.d, fm_n(y), hi);
    *in_planes = 2 * planes;
    return y;
}

static fmap layer(cursor* cur, fmap x, int planes, int n, int stride, int is_aff, int* in_planes, int free_in) {
    for (int b = 0; b < n; ++b) {
        fmap y = block(cur, x, planes, b == 0 ? stride : 1, is_aff, in_planes);
        if (b > 0 || free_in) free(x.d);
        x = y;
    }
    return x;
}

int orc_eres2net_forward(const orc_eres2net* n, const float* feats, int T, float* emb, orc_eres2net_caps* caps) {
    cursor cur = {n, 0};
    const int M = n->m_channels;
    fmap in = {(float*)feats, 1, n->n_mels, T};
    fmap h = next_conv(&cur, in, NULL);
    for (size_t i = 0; i < fm_n(h); ++i) h.d[i] = h.d[i] > 0.0f ? h.d[i] : 0.0f;   /* stem: plain ReLU */
    if (caps && caps->stem) memcpy(caps->stem, h.d, sizeof(float) * fm_n(h));
    int in_planes = M;
    fmap o1 = layer(&cur, h, M, n->num_blocks[0], 1, 0, &in_planes, 1);
    fmap o2 = layer(&cur, o1, M * 2, n->num_blocks[1], 2, 0, &in_planes, 0);
    fmap o1d = next_conv(&cur, o1, NULL);
    free(o1.d);
    fmap f12 = aff(&cur, o2, o1d);
    free(o1d.d);
    fmap o3 = layer(&cur, o2, M * 4, n->num_blocks[2], 2, 1, &in_planes, 0);
    free(o2.d);
    fmap f12d = next_conv(&cur, f12, NULL);
    free(f12.d);
    fmap f123 = aff(&cur, o3, f12d);
    free(f12d.d);
    fmap o4 = layer(&cur, o3, M * 8, n->num_blocks[3], 2, 1, &in_planes, 0);
    free(o3.d);
    fmap f123d = next_conv(&cur, f123, NULL);
    free(f123.d);
    fmap f1234 = aff(&cur, o4, f123d);
    free(o4.d);
    free(f123d.d);
    if (caps && caps->fused) memcpy(caps->fused, f1234.d, sizeof(float) * fm_n(f1234));
    /* TSTP: per (c, h) mean and sqrt(unbiased var + eps) over time (src/encoder_eres2net.cpp:228-242) */
    const int P = 2 * f1234.C * f1234.H;
    float* pooled = malloc(sizeof(float) * (size_t)P);
    orc_tstp(f1234.d, f1234.C, f1234.H, f1234.W, n->var_eps, pooled);
    free(f1234.d);
    if (caps && caps->pooled) memcpy(caps->pooled, pooled, sizeof(float) * (size_t)P);
    orc_linear(pooled, P, n->seg_w, n->seg_b, NULL, n->emb_dim, emb);
    free(pooled);
    if (caps && caps->pre_norm) memcpy(caps->pre_norm, emb, sizeof(float) * (size_t)n->emb_dim);
    if (n->l2_normalize) orc_l2norm(emb, n->emb_dim);
    return cur.idx == n->n_conv ? 0 : 1;
}
