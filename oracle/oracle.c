/*
 * oracle.c - CPU restatement of the reference speaker-embedding path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the parity reference and the CPU
 * baseline, never part of the product library.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------ convolution */

static void out_range(int W, int Wo, int stride, int pad, int off, int* lo, int* hi) {
    /* ow such that 0 <= ow*stride - pad + off <= W-1 (off = kw*dilation) */
    const int a = pad - off;
    *lo = a <= 0 ? 0 : (a + stride - 1) / stride;
    const int b = W - 1 + pad - off;
    *hi = b < 0 ? -1 : b / stride;
    if (*hi > Wo - 1) *hi = Wo - 1;
}

void orc_conv2d_f32_g(const float* x, int IC, int H, int W, const float* w, int OC, int KH, int KW,
                      int sh, int sw, int ph, int pw, int dh, int dw,
                      const float* bias, const float* residual, int relu, float* y) {
    const int Ho = (H + 2 * ph - (KH - 1) * dh - 1) / sh + 1, Wo = (W + 2 * pw - (KW - 1) * dw - 1) / sw + 1;
    float* acc = malloc(sizeof(float) * (Wo > 0 ? Wo : 1));
    for (int oc = 0; oc < OC; ++oc) {
        for (int oh = 0; oh < Ho; ++oh) {
            memset(acc, 0, sizeof(float) * Wo);
            for (int kh = 0; kh < KH; ++kh) {
                const int ih = oh * sh - ph + kh * dh;
                if (ih < 0 || ih >= H) continue;
                for (int kw = 0; kw < KW; ++kw) {
                    int lo, hi;
                    out_range(W, Wo, sw, pw, kw * dw, &lo, &hi);
                    for (int ic = 0; ic < IC; ++ic) {
                        const float wv = w[(((size_t)oc * IC + ic) * KH + kh) * KW + kw];
                        const float* xr = x + ((size_t)ic * H + ih) * W - pw + kw * dw;
                        if (sw == 1) {
                            for (int ow = lo; ow <= hi; ++ow) acc[ow] += wv * xr[ow];
                        } else {
                            for (int ow = lo; ow <= hi; ++ow) acc[ow] += wv * xr[(size_t)ow * sw];
                        }
                    }
                }
            }
            float* yr = y + ((size_t)oc * Ho + oh) * Wo;
            const float* rr = residual ? residual + ((size_t)oc * Ho + oh) * Wo : NULL;
            const float bv = bias ? bias[oc] : 0.0f;
            for (int ow = 0; ow < Wo; ++ow) {
                float v = acc[ow] + bv;
                if (rr) v += rr[ow];
                if (relu && v < 0.0f) v = 0.0f;
                yr[ow] = v;
            }
        }
    }
    free(acc);
}

void orc_conv2d_f32(const float* x, int IC, int H, int W,
                    const float* w, int OC, int KH, int KW, int stride, int pad,
                    const float* bias, const float* residual, int relu, float* y) {
    orc_conv2d_f32_g(x, IC, H, W, w, OC, KH, KW, stride, stride, pad, pad, 1, 1, bias, residual, relu, y);
}

void orc_conv2d_f64_g(const float* x, int IC, int H, int W, const float* w, int OC, int KH, int KW,
                      int sh, int sw, int ph, int pw, int dh, int dw,
                      const float* bias, const float* residual, int relu, double* y) {
    const int Ho = (H + 2 * ph - (KH - 1) * dh - 1) / sh + 1, Wo = (W + 2 * pw - (KW - 1) * dw - 1) / sw + 1;
    for (int oc = 0; oc < OC; ++oc)
        for (int oh = 0; oh < Ho; ++oh)
            for (int ow = 0; ow < Wo; ++ow) {
                double s = 0.0;
                for (int ic = 0; ic < IC; ++ic)
                    for (int kh = 0; kh < KH; ++kh)
                        for (int kw = 0; kw < KW; ++kw) {
                            const int ih = oh * sh - ph + kh * dh, iw = ow * sw - pw + kw * dw;
                            if (ih < 0 || ih >= H || iw < 0 || iw >= W) continue;
                            s += (double)x[((size_t)ic * H + ih) * W + iw] *
                                 (double)w[(((size_t)oc * IC + ic) * KH + kh) * KW + kw];
                        }
                const size_t o = ((size_t)oc * Ho + oh) * Wo + ow;
                if (bias) s += bias[oc];
                if (residual) s += residual[o];
                if (relu && s < 0.0) s = 0.0;
                y[o] = s;
            }
}

void orc_conv2d_f64(const float* x, int IC, int H, int W,
                    const float* w, int OC, int KH, int KW, int stride, int pad,
                    const float* bias, const float* residual, int relu, double* y) {
    orc_conv2d_f64_g(x, IC, H, W, w, OC, KH, KW, stride, stride, pad, pad, 1, 1, bias, residual, relu, y);
}

/* --------------------------------------------------------- pooling and FC */

void orc_tstp(const float* x, int C, int H, int W, float eps, float* pooled) {
    /* src/encoder_resnet.cpp:140-157: mean over time, unbiased var, sqrt(var+eps) */
    const size_t CH = (size_t)C * H;
    for (int c = 0; c < C; ++c)
        for (int h = 0; h < H; ++h) {
            const float* r = x + ((size_t)c * H + h) * W;
            double s = 0.0;
            for (int t = 0; t < W; ++t) s += r[t];
            const float mean = (float)(s / W);
            double s2 = 0.0;
            for (int t = 0; t < W; ++t) { const float d = r[t] - mean; s2 += (double)(d * d); }
            float var = (float)(s2 / W);
            if (W > 1) var *= (float)W / (float)(W - 1);
            pooled[(size_t)c * H + h] = mean;
            pooled[CH + (size_t)c * H + h] = sqrtf(var + eps);
        }
}

void orc_linear(const float* x, int in_dim, const float* w, const float* b,
                const float* mean_vec, int out_dim, float* y) {
    for (int o = 0; o < out_dim; ++o) {
        double s = 0.0;
        const float* r = w + (size_t)o * in_dim;
        for (int i = 0; i < in_dim; ++i) s += (double)r[i] * (double)x[i];
        float v = (float)s;
        if (b) v += b[o];
        if (mean_vec) v -= mean_vec[o];
        y[o] = v;
    }
}

void orc_l2norm(float* v, int n) {
    double n2 = 0.0;
    for (int i = 0; i < n; ++i) n2 += (double)v[i] * (double)v[i];
    const double norm = sqrt(n2);
    if (norm > 0.0)
        for (int i = 0; i < n; ++i) v[i] = (float)((double)v[i] / norm);
}

/* -------------------------------------------------------------- ResNet34 */

int orc_resnet34_forward(const orc_resnet* net, const float* feats, int T,
                         float* emb, orc_resnet_caps* caps) {
    /* src/encoder_resnet.cpp:94-185: stem conv+ReLU, BasicBlocks
     * relu(conv2(relu(conv1(x)+b1))+b2 + shortcut), TSTP, FC, L2. */
    int H = net->n_mels, W = T, C = net->stem_oc;
    size_t cap = (size_t)C * H * W;
    float* x = malloc(sizeof(float) * cap);
    orc_conv2d_f32(feats, 1, H, W, net->stem_w, C, 3, 3, 1, 1, net->stem_b, NULL, 1, x);
    if (caps && caps->stem) memcpy(caps->stem, x, sizeof(float) * (size_t)C * H * W);
    for (int i = 0; i < net->n_blocks; ++i) {
        const int s = net->stride[i], oc = net->out_c[i];
        const int Ho = (H + 2 - 3) / s + 1, Wo = (W + 2 - 3) / s + 1;
        const size_t n = (size_t)oc * Ho * Wo;
        float* h = malloc(sizeof(float) * n);
        float* y = malloc(sizeof(float) * n);
        orc_conv2d_f32(x, C, H, W, net->conv1_w[i], oc, 3, 3, s, 1, net->conv1_b[i], NULL, 1, h);
        float* sc = x;
        float* dn = NULL;
        if (net->down_w[i]) {
            dn = malloc(sizeof(float) * n);
            orc_conv2d_f32(x, C, H, W, net->down_w[i], oc, 1, 1, s, 0, net->down_b[i], NULL, 0, dn);
            sc = dn;
        }
        orc_conv2d_f32(h, oc, Ho, Wo, net->conv2_w[i], oc, 3, 3, 1, 1, net->conv2_b[i], sc, 1, y);
        if (caps && caps->block[i]) memcpy(caps->block[i], y, sizeof(float) * n);
        free(h); free(dn); free(x);
        x = y; C = oc; H = Ho; W = Wo;
    }
    const int P = 2 * C * H;
    float* pooled = malloc(sizeof(float) * P);
    orc_tstp(x, C, H, W, net->var_eps, pooled);
    if (caps && caps->pooled) memcpy(caps->pooled, pooled, sizeof(float) * P);
    orc_linear(pooled, P, net->seg_w, net->seg_b, net->mean_vec, net->emb_dim, emb);
    if (caps && caps->pre_norm) memcpy(caps->pre_norm, emb, sizeof(float) * net->emb_dim);
    if (net->l2_normalize) orc_l2norm(emb, net->emb_dim);
    free(pooled);
    free(x);
    return 0;
}

typedef struct {
    const orc_resnet* net; const orc_fbank_cfg* fcfg;
    const float* pcm; int batch, n_samples, n_threads, tid;
    float* emb;
} job_t;

static void* worker(void* p) {
    job_t* j = p;
    const int T = orc_fbank_frames(j->n_samples, j->fcfg);
    float* feats = malloc(sizeof(float) * (size_t)j->fcfg->n_mels * (T > 0 ? T : 1));
    for (int b = j->tid; b < j->batch; b += j->n_threads) {
        orc_fbank(j->pcm + (size_t)b * j->n_samples, j->n_samples, j->fcfg, feats);
        orc_resnet34_forward(j->net, feats, T, j->emb + (size_t)b * j->net->emb_dim, NULL);
    }
    free(feats);
    return NULL;
}

int orc_embed_batch(const orc_resnet* net, const orc_fbank_cfg* fcfg,
                    const float* pcm, int batch, int n_samples, int n_threads, float* emb) {
    if (orc_fbank_frames(n_samples, fcfg) <= 0) return 1;
    if (n_threads < 1) n_threads = 1;
    if (n_threads > batch) n_threads = batch;
    pthread_t th[256];
    job_t jobs[256];
    if (n_threads > 256) n_threads = 256;
    for (int t = 0; t < n_threads; ++t) {
        jobs[t] = (job_t){net, fcfg, pcm, batch, n_samples, n_threads, t, emb};
        pthread_create(&th[t], NULL, worker, &jobs[t]);
    }
    for (int t = 0; t < n_threads; ++t) pthread_join(th[t], NULL);
    return 0;
}
