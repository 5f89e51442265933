// model_ecapa.cpp - the ECAPA-TDNN encoder of vdk::Model (src/encoder.cpp:299-400).
//
// Layout on the device: every activation is time-major f16 [B][T][C] (the
// NHWC layout of the conv kernels with H = 1, W = T), so a TDNN layer is one
// implicit-GEMM launch with its ReLU and eval BatchNorm in the epilogue:
//   block0     feats -> reflect-padded [B][T+4][96] -> conv k=5 1024
//   block i    tdnn1 (1x1) -> Res2Net groups (k=3 dil i+1 convs with the
//              reflect padding in the conv's input offsets; each group's
//              epilogue also writes the next group's input y_j + x_{j+1})
//              -> tdnn2 (1x1)
//              -> SE (mean -> FC+ReLU -> FC -> sigmoid gate + residual), stored
//              straight into channel slice i-1 of the MFA input `cat`
//   mfa        1x1 over cat
//   ASP        global stats -> per-clip asp.tdnn bias (the [mean; std] columns
//              of the weight, an FC) -> 1x1 over x with ReLU + BN + tanh ->
//              1x1 to f32 logits -> softmax-weighted mean/std
//   head       asp_bn folded into fc on the host -> FC -> L2.
// Weights: f16 [OC][K][IC] for the convs (block0's input channels zero padded
// 80 -> 96), f32 for the SE / ASP-context / fc matrices.
#include <algorithm>
#include <cmath>
#include <functional>
#include <string>

#include "arena.hpp"
#include "common.hpp"
#include "model.hpp"

namespace vdk {

namespace {

constexpr float kBnEps = 1e-5f;     // src/encoder.cpp:121
constexpr float kAspEps = 1e-12f;   // src/encoder.cpp:19

struct ConvShape { int oc, ic, k; };

// ne [K, IC, OC] (F32 conv weight) or [IC, OC] (1x1 stored as a matrix).
ConvShape conv_shape(const GgufFile& g, const std::string& name) {
    const GgufTensor* t = g.tensor(name);
    require(t != nullptr, "voicedetect: missing tensor '" + name + "'");
    if (t->ne.size() == 2) return {(int)t->ne[1], (int)t->ne[0], 1};
    require(t->ne.size() == 3, "voicedetect: conv weight '" + name + "' must be 2-D or 3-D");
    return {(int)t->ne[2], (int)t->ne[1], (int)t->ne[0]};
}

int round_up(int x, int m) { return (x + m - 1) / m * m; }

}  // namespace

void Model::upload_ecapa() {
    const GgufFile& g = *gguf_;
    Ecapa& e = ecapa_;
    ArenaBuilder arena;

    auto f32 = [&](const std::string& name, size_t expect) {
        std::vector<float> v = g.to_f32(name);
        require(v.size() == expect, "voicedetect: tensor '" + name + "' has the wrong size");
        return v;
    };
    // Conv weight [OC][IC][K] -> f16 [OC][K][icp], channels ic..icp zero;
    // input channel i lands at ic_map(i) when given.
    auto layer = [&](const std::string& prefix, int ic_expect, int icp, Layer& l,
                     const std::function<int(int)>& ic_map = nullptr) {
        const std::string wn = prefix + ".weight";
        const ConvShape s = conv_shape(g, wn);
        require(s.ic == ic_expect, "voicedetect: '" + wn + "' has " + std::to_string(s.ic) +
                                       " input channels, expected " + std::to_string(ic_expect));
        require(s.oc % 32 == 0, "voicedetect: '" + wn + "' needs a multiple of 32 output channels");
        const std::vector<float> w = f32(wn, (size_t)s.oc * s.ic * s.k);
        std::vector<uint16_t> packed((size_t)s.oc * s.k * icp, 0);
        for (int o = 0; o < s.oc; ++o)
            for (int i = 0; i < s.ic; ++i)
                for (int k = 0; k < s.k; ++k)
                    packed[((size_t)o * s.k + k) * icp + (ic_map ? ic_map(i) : i)] =
                        float_to_half_bits(w[((size_t)o * s.ic + i) * s.k + k]);
        l.ic = icp; l.oc = s.oc; l.k = s.k;
        arena.put(packed, &l.w);
        arena.put(f32(prefix + ".bias", (size_t)s.oc), &l.b);
        return s;
    };
    // Eval BatchNorm -> scale, shift (src/encoder.cpp:110-150).
    auto bn = [&](const std::string& p, int c, Layer& l) {
        const std::vector<float> gam = f32(p + ".weight", c), bet = f32(p + ".bias", c),
                                 mu = f32(p + ".running_mean", c), var = f32(p + ".running_var", c);
        std::vector<float> sc(c), sh(c);
        for (int i = 0; i < c; ++i) {
            sc[i] = gam[i] / std::sqrt(var[i] + kBnEps);
            sh[i] = bet[i] - sc[i] * mu[i];
        }
        arena.put(sc, &l.scale);
        arena.put(sh, &l.shift);
    };

    // block0: Conv1d(n_mels -> C, k) -> ReLU -> BN
    e.n_mels = cfg_.fbank.n_mels;
    e.c_pad0 = round_up(e.n_mels, 32);
    const ConvShape s0 = layer("blocks.0.conv.conv", e.n_mels, e.c_pad0, e.block0);
    require(s0.k % 2 == 1, "voicedetect: block0 kernel size must be odd");
    bn("blocks.0.norm.norm", s0.oc, e.block0);
    e.C = s0.oc;
    const int C = e.C;

    // SE-Res2Net blocks: count and scale from the manifest (src/encoder.cpp:335-338, 237-240)
    // (ArenaBuilder keeps the addresses of the pointer fields: size the block
    // list first so that no element moves afterwards.)
    int n_blocks = 0;
    while (g.tensor("blocks." + std::to_string(n_blocks + 1) + ".tdnn1.conv.conv.weight")) ++n_blocks;
    require(n_blocks > 0, "voicedetect: ECAPA model has no SE-Res2Net blocks");
    e.blocks.assign(n_blocks, EcapaBlock());
    for (int i = 1; i <= n_blocks; ++i) {
        const std::string p = "blocks." + std::to_string(i);
        EcapaBlock& b = e.blocks[i - 1];
        b.dil = i + 1;
        layer(p + ".tdnn1.conv.conv", C, C, b.tdnn1);
        require(b.tdnn1.oc == C, "voicedetect: " + p + ".tdnn1 must keep the channel count");
        bn(p + ".tdnn1.norm.norm", C, b.tdnn1);
        int scale = 1;
        while (g.tensor(p + ".res2net_block.blocks." + std::to_string(scale - 1) + ".conv.conv.weight")) ++scale;
        require(scale >= 2 && C % scale == 0, "voicedetect: " + p + " Res2Net scale must divide the channels");
        if (i == 1) e.scale = scale;
        require(scale == e.scale, "voicedetect: Res2Net scale differs between blocks");
        const int grp = C / scale;
        require(grp % 32 == 0, "voicedetect: Res2Net group width must be a multiple of 32");
        b.res.resize(scale - 1);
        for (int j = 0; j < scale - 1; ++j) {
            const std::string q = p + ".res2net_block.blocks." + std::to_string(j);
            const ConvShape sj = layer(q + ".conv.conv", grp, grp, b.res[j]);
            require(sj.oc == grp && sj.k == 3, "voicedetect: " + q + " must be a k=3 conv of the group width");
            bn(q + ".norm.norm", grp, b.res[j]);
        }
        // tdnn2 reads the Res2Net output slots in the order [y_1 | x_0 | y_2 .. y_{scale-1}]
        // (encode_ecapa): input channel groups 0 and 1 swap
        layer(p + ".tdnn2.conv.conv", C, C, b.tdnn2, [grp](int c) {
            return c < grp ? c + grp : (c < 2 * grp ? c - grp : c);
        });
        require(b.tdnn2.oc == C, "voicedetect: " + p + ".tdnn2 must keep the channel count");
        bn(p + ".tdnn2.norm.norm", C, b.tdnn2);
        const ConvShape se1 = conv_shape(g, p + ".se_block.conv1.conv.weight");
        require(se1.ic == C && se1.k == 1, "voicedetect: " + p + ".se_block.conv1 must be 1x1 over C");
        b.se_ch = se1.oc;
        arena.put(f32(p + ".se_block.conv1.conv.weight", (size_t)b.se_ch * C), &b.se1_w);
        arena.put(f32(p + ".se_block.conv1.conv.bias", b.se_ch), &b.se1_b);
        arena.put(f32(p + ".se_block.conv2.conv.weight", (size_t)C * b.se_ch), &b.se2_w);
        arena.put(f32(p + ".se_block.conv2.conv.bias", C), &b.se2_b);
    }
    e.group = C / e.scale;
    const int nb = (int)e.blocks.size();

    // MFA over the concatenated block outputs
    const ConvShape sm = layer("mfa.conv.conv", nb * C, nb * C, e.mfa_l);
    require(sm.k == 1, "voicedetect: mfa must be 1x1");
    bn("mfa.norm.norm", sm.oc, e.mfa_l);
    e.mfa = sm.oc;
    const int M = e.mfa;

    // ASP: asp.tdnn weight [att][3M] split into the x columns (conv) and the
    // [mean; std] columns (per-clip FC).
    const ConvShape sa = conv_shape(g, "asp.tdnn.conv.conv.weight");
    require(sa.ic == 3 * M && sa.k == 1 && sa.oc % 32 == 0, "voicedetect: asp.tdnn must be 1x1 over 3*mfa");
    e.att = sa.oc;
    {
        const std::vector<float> w = f32("asp.tdnn.conv.conv.weight", (size_t)e.att * 3 * M);
        std::vector<uint16_t> wx((size_t)e.att * M);
        std::vector<float> ws((size_t)e.att * 2 * M);
        for (int o = 0; o < e.att; ++o) {
            for (int i = 0; i < M; ++i) wx[(size_t)o * M + i] = float_to_half_bits(w[(size_t)o * 3 * M + i]);
            for (int i = 0; i < 2 * M; ++i) ws[(size_t)o * 2 * M + i] = w[(size_t)o * 3 * M + M + i];
        }
        e.asp_x.ic = M; e.asp_x.oc = e.att; e.asp_x.k = 1;
        arena.put(wx, &e.asp_x.w);
        arena.put(ws, &e.asp_stats_w);
        arena.put(f32("asp.tdnn.conv.conv.bias", e.att), &e.asp_b);
        bn("asp.tdnn.norm.norm", e.att, e.asp_x);
    }
    const ConvShape sc = layer("asp.conv.conv", e.att, e.att, e.asp_conv);
    require(sc.oc == M && sc.k == 1, "voicedetect: asp.conv must be 1x1 att -> mfa");

    // asp_bn folded into fc: W' = W diag(s), b' = b + W t (double accumulation)
    const ConvShape sf = conv_shape(g, "fc.conv.weight");
    require(sf.ic == 2 * M && sf.k == 1 && sf.oc == cfg_.embedding_dim,
            "voicedetect: fc.conv must be 1x1 from 2*mfa to embedding_dim");
    {
        const int P = 2 * M, E = sf.oc;
        const std::vector<float> w = f32("fc.conv.weight", (size_t)E * P), b = f32("fc.conv.bias", E);
        const std::vector<float> gam = f32("asp_bn.norm.weight", P), bet = f32("asp_bn.norm.bias", P),
                                 mu = f32("asp_bn.norm.running_mean", P), var = f32("asp_bn.norm.running_var", P);
        std::vector<float> wf((size_t)E * P), bf(E);
        for (int o = 0; o < E; ++o) {
            double acc = b[o];
            for (int i = 0; i < P; ++i) {
                const float s = gam[i] / std::sqrt(var[i] + kBnEps);
                const float t = bet[i] - s * mu[i];
                wf[(size_t)o * P + i] = w[(size_t)o * P + i] * s;
                acc += (double)w[(size_t)o * P + i] * t;
            }
            bf[o] = (float)acc;
        }
        arena.put(wf, &e.fc_w);
        arena.put(bf, &e.fc_b);
    }
    pooled_dim_ = 2 * M;
    arena_ = arena.upload();
}

void Model::alloc_ecapa_workspace(int batch, int T) {
    const Ecapa& e = ecapa_;
    Workspace& w = ws_;
    const size_t BT = (size_t)batch * T;
    const int pad0 = (e.block0.k - 1) / 2;
    size_t fc_work = vdk_linear_workspace_size(batch, 2 * e.mfa, cfg_.embedding_dim);
    fc_work = std::max(fc_work, vdk_linear_workspace_size(batch, 2 * e.mfa, e.att));
    for (const EcapaBlock& b : e.blocks) {
        fc_work = std::max(fc_work, vdk_linear_workspace_size(batch, e.C, b.se_ch));
        fc_work = std::max(fc_work, vdk_linear_workspace_size(batch, b.se_ch, e.C));
    }
    const int nb = (int)e.blocks.size();
    int se_max = 0;
    for (const EcapaBlock& b : e.blocks) se_max = std::max(se_max, b.se_ch);
    w.x0p = ws_alloc(2 * (size_t)batch * (T + 2 * pad0) * e.c_pad0);
    w.h0 = ws_alloc(2 * BT * e.C);
    w.t1 = ws_alloc(2 * BT * (e.C + e.group));   // scale + 1 group slots per frame
    w.s2b[0] = ws_alloc(2 * BT * e.group);
    w.s2b[1] = ws_alloc(2 * BT * e.group);
    w.t2 = ws_alloc(2 * BT * e.C);
    w.cat = ws_alloc(2 * BT * nb * e.C);
    w.mfa = ws_alloc(2 * BT * e.mfa);
    w.a1 = ws_alloc(2 * BT * e.att);
    if (!(e.att == 128 && e.mfa % 64 == 0)) w.logits = static_cast<float*>(ws_alloc(4 * BT * e.mfa));
    w.se_m = static_cast<float*>(ws_alloc(4 * (size_t)batch * e.C));
    w.se_h = static_cast<float*>(ws_alloc(4 * (size_t)batch * se_max));
    w.se_g = static_cast<float*>(ws_alloc(4 * (size_t)batch * e.C));
    w.stats = static_cast<float*>(ws_alloc(4 * (size_t)batch * 2 * e.mfa));
    w.pb = static_cast<float*>(ws_alloc(4 * (size_t)batch * e.att));
    w.fc_work_bytes = fc_work;
    w.fc_work = ws_alloc(fc_work);
}

void Model::tdnn(const char* name, const Layer& l, const void* x, int x_stride, int batch, int W, int dil,
                 const float* bias, int bias_bs, int relu, int tanh_after, void* y, int y_stride, int y_f32) {
    const int Wo = W - (l.k - 1) * dil;
    if (profiling_) {
        const double npix = (double)batch * Wo;
        const double flops = 2.0 * l.k * l.ic * l.oc * npix;
        const double bytes = 2.0 * ((double)batch * W * l.ic + (double)l.oc * l.k * l.ic) +
                             npix * l.oc * (y_f32 ? 4.0 : 2.0);
        prof_begin((std::string("conv.") + name).c_str(), flops, bytes);
    }
    vdk_conv_desc d{};
    d.x = x; d.batch = batch; d.H = 1; d.W = W; d.IC = l.ic; d.x_stride = x_stride;
    d.w = l.w; d.OC = l.oc; d.KH = 1; d.KW = l.k;
    d.stride_h = d.stride_w = 1; d.dil_h = 1; d.dil_w = dil;
    d.bias = bias; d.bias_batch_stride = bias_bs;
    d.post_scale = l.scale; d.post_shift = l.shift;
    d.act = relu ? VDK_ACT_RELU : VDK_ACT_NONE; d.tanh_after = tanh_after;
    d.y = y; d.y_stride = y_stride; d.y_f32 = y_f32;
    d.tile = -1;
    check_rc(vdk_conv2d_ex(&d, stream_));
    prof_end();
}

// One Res2Net group conv: k=3 dilated over T frames with SpeechBrain's
// reflect padding (src/encoder.cpp:32-52) folded into the conv's input
// offsets, + bias -> ReLU -> BN; y2 (optional) = that output + r2 (the next
// group's input).
void Model::res2_conv(const Layer& l, const void* x, int x_stride, int batch, int T, int dil, void* y, int y_stride,
                      const void* r2, int r2_stride, void* y2) {
    if (profiling_) {
        const double npix = (double)batch * T;
        const double bytes = 2.0 * (npix * l.ic + (double)l.oc * l.k * l.ic) + npix * l.oc * (y2 ? 6.0 : 2.0);
        prof_begin("conv.ecapa_res2_conv", 2.0 * l.k * l.ic * l.oc * npix, bytes);
    }
    vdk_conv_desc d{};
    d.x = x; d.batch = batch; d.H = 1; d.W = T; d.IC = l.ic; d.x_stride = x_stride;
    d.w = l.w; d.OC = l.oc; d.KH = 1; d.KW = l.k;
    d.stride_h = d.stride_w = 1; d.dil_h = 1; d.dil_w = dil;
    d.pad_w = (l.k - 1) / 2 * dil; d.reflect_pad = 1;
    d.bias = l.b;
    d.post_scale = l.scale; d.post_shift = l.shift;
    d.act = VDK_ACT_RELU;
    d.y = y; d.y_stride = y_stride;
    d.y2 = y2; d.y2_stride = l.oc; d.res2 = r2; d.res2_stride = r2_stride;
    d.tile = -1;
    check_rc(vdk_conv2d_ex(&d, stream_));
    prof_end();
}

void Model::linear(const char* name, const float* x, int batch, int in_dim, const float* w, const float* b,
                   const float* mv, int out_dim, int relu, float* y) {
    prof_begin(name, 2.0 * batch * (double)in_dim * out_dim,
               4.0 * ((double)batch * in_dim + (double)in_dim * out_dim + (double)batch * out_dim));
    check_rc(vdk_linear_ex(x, batch, in_dim, w, b, mv, out_dim, relu, y, ws_.fc_work, ws_.fc_work_bytes, stream_));
    prof_end();
}

void Model::encode_ecapa(int batch, int T) {
    const Ecapa& e = ecapa_;
    Workspace& w = ws_;
    const int C = e.C, G = e.group, M = e.mfa, nb = (int)e.blocks.size();
    const int catS = nb * C;
    const size_t gB = 2 * (size_t)G;   // bytes per group slice

    // block0: reflect pad (k-1)/2, time-major, zero channels to c_pad0
    const int pad0 = (e.block0.k - 1) / 2;
    prof_begin("ecapa_feats_tmajor", 0.0, 4.0 * batch * (double)e.n_mels * T + 2.0 * batch * (T + 2.0 * pad0) * e.c_pad0);
    check_rc(vdk_feats_tmajor(w.feats, w.fb_mean, batch, e.n_mels, T, pad0, e.c_pad0, w.x0p, stream_));
    prof_end();
    tdnn("ecapa_block0", e.block0, w.x0p, e.c_pad0, batch, T + 2 * pad0, 1, e.block0.b, 0, 1, 0, w.h0, C, 0);

    for (int i = 0; i < nb; ++i) {
        const EcapaBlock& b = e.blocks[i];
        const void* xin = i == 0 ? w.h0 : static_cast<const uint8_t*>(w.cat) + 2 * (size_t)(i - 1) * C;
        const int xs = i == 0 ? C : catS;
        // t1 holds scale + 1 group slots per frame (stride S = C + G): tdnn1
        // writes x_0 .. x_{scale-1} to slots 1 .. scale; group j reads its
        // input (x_1 from slot 2, then y_{j-1} + x_j from s2b[j & 1]) with the
        // reflect padding done by the conv, writes y_j to slot j (group 1:
        // slot 0), whose x_{j-1} every earlier launch has consumed, and, for
        // j < scale - 1, y_j + x_{j+1} to s2b[(j + 1) & 1]; tdnn2 then reads
        // slots 0 .. scale-1 = [y_1 | x_0 | y_2 .. y_{scale-1}] (its weight
        // columns permuted to match) (src/encoder.cpp:174-200).
        const int S = C + G;
        uint8_t* t1 = static_cast<uint8_t*>(w.t1);
        tdnn("ecapa_tdnn1", b.tdnn1, xin, xs, batch, T, 1, b.tdnn1.b, 0, 1, 0, t1 + gB, S, 0);
        if (G == 128 && e.scale <= 8 && (e.scale - 1) * b.dil <= 64) {
            // all groups in one launch per time tile, the same bits as the chain below
            vdk_res2_weights rw{};
            for (int j = 0; j + 1 < e.scale; ++j) {
                rw.w[j] = b.res[j].w;
                rw.bias[j] = b.res[j].b;
                rw.scale[j] = b.res[j].scale;
                rw.shift[j] = b.res[j].shift;
            }
            if (profiling_) {
                const double npix = (double)batch * T, n = e.scale - 1.0;
                prof_begin("conv.ecapa_res2_block", n * 2.0 * 3 * G * G * npix,
                           2.0 * npix * G * (2.0 * n) + n * 2.0 * 3 * G * G);
            }
            check_rc(vdk_res2_block(w.t1, S, batch, T, G, e.scale, b.dil, &rw, stream_));
            prof_end();
        } else {
            for (int j = 1; j < e.scale; ++j) {
                const bool last = j + 1 == e.scale;
                const void* in = j == 1 ? static_cast<const void*>(t1 + 2 * gB) : w.s2b[j & 1];
                res2_conv(b.res[j - 1], in, j == 1 ? S : G, batch, T, b.dil, t1 + (j == 1 ? 0 : j) * gB, S,
                          last ? nullptr : t1 + (j + 2) * gB, S, last ? nullptr : w.s2b[(j + 1) & 1]);
            }
        }
        tdnn("ecapa_tdnn2", b.tdnn2, w.t1, S, batch, T, 1, b.tdnn2.b, 0, 1, 0, w.t2, C, 0);
        // SE (src/encoder.cpp:207-219) and the residual (src/encoder.cpp:243)
        prof_begin("ecapa_se_mean", 0.0, 2.0 * batch * (double)T * C);
        check_rc(vdk_channel_mean(w.t2, C, batch, T, C, w.se_m, stream_));
        prof_end();
        linear("ecapa_se_fc1", w.se_m, batch, C, b.se1_w, b.se1_b, nullptr, b.se_ch, 1, w.se_h);
        // the sigmoid once per (clip, channel) in fc2's reduce
        linear("ecapa_se_fc2", w.se_h, batch, b.se_ch, b.se2_w, b.se2_b, nullptr, C, VDK_ACT_SIGMOID, w.se_g);
        void* out = static_cast<uint8_t*>(w.cat) + 2 * (size_t)i * C;
        prof_begin("ecapa_se_gate", 0.0, 6.0 * batch * (double)T * C);
        check_rc(vdk_se_scale_residual(w.t2, C, w.se_g, xin, xs, batch, T, C, out, catS, stream_));
        prof_end();
    }

    tdnn("ecapa_mfa", e.mfa_l, w.cat, catS, batch, T, 1, e.mfa_l.b, 0, 1, 0, w.mfa, M, 0);

    // Attentive statistics pooling (src/encoder.cpp:262-295)
    prof_begin("ecapa_asp_stats", 0.0, 4.0 * batch * (double)T * M);
    check_rc(vdk_asp_stats(w.mfa, M, batch, T, M, kAspEps, w.stats, stream_));
    prof_end();
    linear("ecapa_asp_ctx", w.stats, batch, 2 * M, e.asp_stats_w, e.asp_b, nullptr, e.att, 0, w.pb);
    tdnn("ecapa_asp_tdnn", e.asp_x, w.mfa, M, batch, T, 1, w.pb, e.att, 1, 1, w.a1, e.att, 0);
    if (e.att == 128 && M % 64 == 0) {
        // the asp.conv logits and the pooling in one launch (logits stay on chip)
        prof_begin("ecapa_asp_attn_pool", 2.0 * batch * (double)T * M * e.att, 2.0 * batch * (double)T * (M + e.att) * 2);
        check_rc(vdk_asp_attn_pool(w.a1, e.att, e.asp_conv.w, e.asp_conv.b, e.att, w.mfa, M, batch, T, M, kAspEps,
                                   w.pooled, stream_));
        prof_end();
    } else {
        tdnn("ecapa_asp_conv", e.asp_conv, w.a1, e.att, batch, T, 1, e.asp_conv.b, 0, 0, 0, w.logits, M, 1);
        prof_begin("ecapa_asp_pool", 0.0, 4.0 * batch * (double)T * M * 2 + 2.0 * batch * (double)T * M * 2);
        check_rc(vdk_asp_pool(w.logits, M, w.mfa, M, batch, T, M, kAspEps, w.pooled, stream_));
        prof_end();
    }

    embed_fc("ecapa_fc", w.pooled, batch, 2 * M, e.fc_w, e.fc_b, nullptr, cfg_.embedding_dim);
}

}  // namespace vdk
