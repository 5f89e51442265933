/*
 * oracle.h - CPU restatement of the reference speaker-embedding path.
 *
 * TEST INFRASTRUCTURE ONLY.  The HIP implementation's results are compared
 * against this library: only the test suite, the smoke check and the CPU-baseline
 * leg of the benchmark may load it.  The product library never links it and
 * has no CPU fallback.
 *
 * Every function restates one reference function (cited per declaration) in
 * plain C with the reference's arithmetic precision: FBank in double with
 * float framing steps, convolutions/pooling/FC in f32 (plus an f64 brute-force
 * convolution used to pin the f32 one), L2 norm accumulated in double.
 *
 * Layouts follow the reference (ggml ne fastest-first, written here
 * slowest-first): feature maps are NCHW per clip [C][H=freq][W=time],
 * conv weights [OC][IC][KH][KW], FC weights [OUT][IN].
 *
 * Parity pins (tests/): FBank against golden vectors produced by the
 * reference's own src/fbank.cpp, closed forms (frame count, povey window, mel
 * filter edges, CMN zero-mean) and a naive DFT; convolutions against the f64
 * brute force and the reference test_blocked.cpp cases; pooling/FC/L2 against
 * closed forms.  No function is "parity unpinned".
 */
#ifndef VD_ORACLE_H
#define VD_ORACLE_H

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int sample_rate, n_mels, n_fft, win_length, hop_length;
    float preemph, low_freq, high_freq; /* high_freq <= 0 means Nyquist */
    int cmn;
} orc_fbank_cfg;

/* Frame count with snip_edges framing (src/fbank.cpp:130). */
int orc_fbank_frames(int n_samples, const orc_fbank_cfg* cfg);

/* Kaldi FBank + CMN (src/fbank.cpp:121-205).  out: feat-major [n_mels][T].
 * Returns T (0 if the clip is shorter than one window). */
int orc_fbank(const float* pcm, int n_samples, const orc_fbank_cfg* cfg, float* out);

/* Power spectrum |X_k|^2, k = 0..n_fft/2, of a real frame zero-padded to
 * n_fft (src/fbank.cpp:92-118).  use_dft=1 forces the naive O(N^2) DFT. */
void orc_powspec(const float* frame, int frame_len, int n_fft, int use_dft, double* out);

/* Kaldi triangular mel filter matrix [n_mels][n_fft/2+1] (src/fbank.cpp:140-158). */
void orc_mel_filters(const orc_fbank_cfg* cfg, double* fb);

/* Povey window (src/fbank.cpp:132-135). */
void orc_povey_window(int win, double* w);

/* 2D convolution, one clip, NCHW f32 (src/directconv.cpp blocked island
 * contract: zero padding, f32 accumulation in (kh, kw, ic) order).
 * y = conv(x, w) + bias; if residual: y += residual; if relu: y = max(y, 0).
 * bias / residual may be NULL.  Output [OC][Ho][Wo] with
 * Ho = (H + 2*pad - KH)/stride + 1. */
void orc_conv2d_f32(const float* x, int IC, int H, int W,
                    const float* w, int OC, int KH, int KW, int stride, int pad,
                    const float* bias, const float* residual, int relu, float* y);

/* General form: separate strides / zero pads / dilations per axis
 * (Ho = (H + 2*ph - (KH-1)*dh - 1)/sh + 1).  The CAM++ FCM strides only the
 * frequency axis (src/encoder_campplus.cpp:67-76); its 1-D convs are H = 1. */
void orc_conv2d_f32_g(const float* x, int IC, int H, int W, const float* w, int OC, int KH, int KW,
                      int sh, int sw, int ph, int pw, int dh, int dw,
                      const float* bias, const float* residual, int relu, float* y);
void orc_conv2d_f64_g(const float* x, int IC, int H, int W, const float* w, int OC, int KH, int KW,
                      int sh, int sw, int ph, int pw, int dh, int dw,
                      const float* bias, const float* residual, int relu, double* y);

/* Same contract, every product and sum in double (the brute-force pin). */
void orc_conv2d_f64(const float* x, int IC, int H, int W,
                    const float* w, int OC, int KH, int KW, int stride, int pad,
                    const float* bias, const float* residual, int relu, double* y);

/* Temporal statistics pooling (src/encoder_resnet.cpp:140-157): per (c, h)
 * mean over W and sqrt(unbiased var + eps); pooled = [mean(c,h) ; std(c,h)]
 * flattened C-outer / H-inner, length 2*C*H. */
void orc_tstp(const float* x, int C, int H, int W, float eps, float* pooled);

/* y = W x + b - mean_vec (src/encoder_resnet.cpp:159-169); b / mean_vec may be NULL. */
void orc_linear(const float* x, int in_dim, const float* w, const float* b,
                const float* mean_vec, int out_dim, float* y);

/* In-place L2 normalisation accumulated in double; skipped if the norm is 0
 * (src/encoder_resnet.cpp:177-183). */
void orc_l2norm(float* v, int n);

#define ORC_MAX_BLOCKS 32

/* WeSpeaker ResNet34 weights (src/encoder_resnet.cpp, model_loader.hpp:48-58),
 * dequantised to f32.  down_w[i] == NULL means an identity shortcut. */
typedef struct {
    int n_mels, stem_oc;
    const float* stem_w; const float* stem_b;
    int n_blocks;
    int in_c[ORC_MAX_BLOCKS], out_c[ORC_MAX_BLOCKS], stride[ORC_MAX_BLOCKS];
    const float* conv1_w[ORC_MAX_BLOCKS]; const float* conv1_b[ORC_MAX_BLOCKS];
    const float* conv2_w[ORC_MAX_BLOCKS]; const float* conv2_b[ORC_MAX_BLOCKS];
    const float* down_w[ORC_MAX_BLOCKS];  const float* down_b[ORC_MAX_BLOCKS];
    const float* seg_w; const float* seg_b; const float* mean_vec;
    int emb_dim;
    float var_eps;
    int l2_normalize;
} orc_resnet;

/* Optional per-stage captures (NCHW f32, caller-sized); any pointer may be NULL. */
typedef struct {
    float* stem;          /* [stem_oc][n_mels][T] after ReLU */
    float* block[ORC_MAX_BLOCKS]; /* each block's output */
    float* pooled;        /* [2*C*H'] */
    float* pre_norm;      /* [emb_dim] */
} orc_resnet_caps;

/* Full ResNet34 forward of one clip from FBank features [n_mels][T]
 * (src/encoder_resnet.cpp:94-185).  Returns 0 on success. */
int orc_resnet34_forward(const orc_resnet* net, const float* feats, int T,
                         float* emb, orc_resnet_caps* caps);

/* PCM -> FBank -> ResNet34 -> embedding for `batch` clips of n_samples each,
 * clip-parallel over n_threads threads.  emb: [batch][emb_dim].  Returns 0. */
int orc_embed_batch(const orc_resnet* net, const orc_fbank_cfg* fcfg,
                    const float* pcm, int batch, int n_samples, int n_threads, float* emb);

/* ------------------------------------------------------------ ECAPA-TDNN */

/* Conv1d weight [oc][ic][k] and bias [oc] (src/encoder.cpp:62-109). */
typedef struct { const float* w; const float* b; int oc, ic, k; } orc_conv1d;
/* Eval BatchNorm1d parameters (src/encoder.cpp:125-151, eps 1e-5). */
typedef struct { const float* gamma; const float* beta; const float* mean; const float* var; int c; } orc_bn;

#define ORC_MAX_RES 8
#define ORC_MAX_SCALE 16

typedef struct {
    int n_mels, channels, scale, n_res, mfa_ch, emb_dim, l2_normalize;
    orc_conv1d block0; orc_bn bn0;
    orc_conv1d tdnn1[ORC_MAX_RES], tdnn2[ORC_MAX_RES], se1[ORC_MAX_RES], se2[ORC_MAX_RES];
    orc_bn bn_t1[ORC_MAX_RES], bn_t2[ORC_MAX_RES];
    orc_conv1d res[ORC_MAX_RES][ORC_MAX_SCALE]; orc_bn bn_res[ORC_MAX_RES][ORC_MAX_SCALE];
    orc_conv1d mfa; orc_bn bn_mfa;
    orc_conv1d asp_tdnn; orc_bn bn_asp; orc_conv1d asp_conv; orc_bn asp_bn;
    orc_conv1d fc;
} orc_ecapa;

typedef struct {
    float* block[ORC_MAX_RES + 1];   /* block0 .. block n_res outputs, [C][T] */
    float* mfa;                      /* [mfa_ch][T] */
    float* pooled;                   /* [2*mfa_ch] raw ASP output (before asp_bn) */
    float* pre_norm;                 /* [emb_dim] */
} orc_ecapa_caps;

/* Reflect-padded ("same") dilated conv1d, stride 1: x [ic][T] -> y [oc][T]
 * (src/encoder.cpp:32-109: pad (k-1)/2*dil, reflect without edge repeat). */
void orc_conv1d_same(const float* x, int T, const orc_conv1d* c, int dilation, float* y);
/* y = x * g/sqrt(var+eps) + (beta - mean*g/sqrt(var+eps)), x [C][T] in place. */
void orc_bn_apply(float* x, int T, const orc_bn* bn);
/* Attentive statistics pooling with global context (src/encoder.cpp:262-295):
 * x [C][T] -> pooled [2C] = [mu ; sd]. */
void orc_ecapa_asp(const orc_ecapa* net, const float* x, int T, float* pooled);
/* Full ECAPA forward of one clip from FBank features [n_mels][T]
 * (src/encoder.cpp:299-400). Returns 0. */
int orc_ecapa_forward(const orc_ecapa* net, const float* feats, int T, float* emb, orc_ecapa_caps* caps);

/* ---------------------------------------------------------------- CAM++ */

/* One conv in manifest order: weight [oc][ic][kh][kw] (1-D convs kh = 1,
 * 1x1 kh = kw = 1), bias may be NULL. */
typedef struct { const float* w; const float* b; int oc, ic, kh, kw; } orc_conv;

#define ORC_CAMPP_MAX_CONV 256
#define ORC_CAMPP_MAX_BN 64

/* 3D-Speaker CAM++ from its flat execution-order manifests
 * (model_loader.hpp:82-99): conv[] in forward order, bn[] the affine BNs in
 * forward order, emb_mean/emb_var the final affine-free BN. */
typedef struct {
    int n_mels, n_conv, n_bn, l2_normalize;
    float bn_eps;
    orc_conv conv[ORC_CAMPP_MAX_CONV];
    orc_bn bn[ORC_CAMPP_MAX_BN];
    const float* emb_mean; const float* emb_var;
} orc_campplus;

typedef struct {
    float* fcm;        /* [C*H'][T] FCM output, channel c*H' + h */
    float* tdnn;       /* [128][T'] */
    float* block[3];   /* transit outputs [C_b][T'] */
    float* pooled;     /* [2C] mean ; unbiased std */
    float* pre_norm;   /* [emb] */
} orc_campplus_caps;

/* Full CAM++ forward of one clip from FBank features [n_mels][T]
 * (src/encoder_campplus.cpp:148-320).  Returns 0, or 1 when the manifest does
 * not match the fixed topology. */
int orc_campplus_forward(const orc_campplus* net, const float* feats, int T, float* emb,
                         orc_campplus_caps* caps);

/* ------------------------------------------------------------- ERes2Net */

#define ORC_ERES_MAX_CONV 128

/* 3D-Speaker ERes2Net from its flat execution-order manifest
 * (model_loader.hpp:68-79): conv[] with per-conv stride[], blocks per layer,
 * m_channels, the Res2Net scale, the seg_1 embedding FC. */
typedef struct {
    int n_mels, n_conv, m_channels, scale, emb_dim, l2_normalize;
    int num_blocks[4];
    float relu_clamp, var_eps;
    orc_conv conv[ORC_ERES_MAX_CONV];
    int stride[ORC_ERES_MAX_CONV];
    const float* seg_w; const float* seg_b;
} orc_eres2net;

typedef struct {
    float* stem;       /* [M][n_mels][T] after ReLU */
    float* fused;      /* [16M][H'][W'] the last AFF output */
    float* pooled;     /* [2 * 16M * H'] */
    float* pre_norm;   /* [emb] */
} orc_eres2net_caps;

/* Full ERes2Net forward of one clip from FBank features [n_mels][T]
 * (src/encoder_eres2net.cpp:139-265).  Returns 0, or 1 when the manifest
 * does not match the topology. */
int orc_eres2net_forward(const orc_eres2net* net, const float* feats, int T, float* emb,
                         orc_eres2net_caps* caps);

#ifdef __cplusplus
}
#endif
#endif
