// model_w2v2.cpp - the wav2vec2 analyze models of vdk::Model
// (src/analyze_w2v2.cpp, src/model.cpp:80-101).
//
// Layout on the device: every activation is time-major [B][T][C] (f16 for
// GEMM operands, f32 where a LayerNorm or the residual stream reads it), so
// each conv / linear layer is one implicit-GEMM launch (H = 1, W = T):
//   conv0      raw waveform [(normalize)] -> k10 s5 1 -> C0, GroupNorm or
//              LayerNorm, GELU (vdk_w2v2_conv0)
//   conv 1..   k x C -> C stride s, GELU in the epilogue ("group"), or bias ->
//              f32 -> LayerNorm + GELU ("layer")
//   projection LayerNorm(C) -> 1x1 C -> H (+bias)
//   pos conv   per group: k128 pad 64 conv over its H/groups channels, bias,
//              GELU, + projection (residual after the activation), last step
//              dropped (out_w = T) -> f32 residual stream
//   layers     post-norm (base): h = LN(h + out(attn(qkv(h)))), h = LN(h + ff(h));
//              pre-norm (large-robust): r += out(attn(qkv(LN(r)))), r += ff(LN(r)),
//              final LN.  q/k/v is one GEMM over stacked weights.
//   heads      emotion: weighted layer sum -> time mean -> projector ->
//              classifier; age/gender: time mean of the last state -> two
//              dense+tanh -> out_proj heads.
// The emotion head takes the time mean of each hidden state and sums those
// with the layer weights, then applies the projector: the reference sums the
// states frame by frame, projects every frame and then takes the time mean
// (src/analyze_w2v2.cpp:528-550), and mean_t(W sum_i w_i x_it + b) =
// W sum_i w_i mean_t(x_it) + b since every step is linear.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <string>

#include "arena.hpp"
#include "audio.hpp"
#include "common.hpp"
#include "model.hpp"

namespace vdk {

namespace {
constexpr float kGroupNormEps = 1e-5f;   // src/analyze_w2v2.cpp:57-60
constexpr float kWaveNormEps = 1e-7f;    // src/analyze_w2v2.cpp:63-70
}  // namespace

bool Model::is_analyzer() const {
    return cfg_.arch == "wav2vec2_emotion" || cfg_.arch == "wav2vec2_age_gender";
}

int Model::analyze_outputs() const {
    if (!is_analyzer()) return 0;
    if (cfg_.arch == "wav2vec2_age_gender") return 1 + (int)cfg_.gender_labels.size();
    return (int)cfg_.emotion_labels.size();
}

int Model::analyze_frames(int n) const {
    const W2v2Cfg& c = cfg_.w2v2;
    int t = n;
    for (size_t i = 0; i < c.conv_kernels.size(); ++i) {
        const int k = c.conv_kernels[i], s = c.conv_strides[i];
        if (t < k || s <= 0) return 0;
        t = (t - k) / s + 1;
    }
    return t;
}

void Model::upload_w2v2() {
    const GgufFile& g = *gguf_;
    const W2v2Cfg& c = cfg_.w2v2;
    W2v2& m = w2_;
    ArenaBuilder arena;
    const bool age_gender = cfg_.arch == "wav2vec2_age_gender";
    const bool layer_fe = c.feat_extract_norm == "layer", group_fe = c.feat_extract_norm == "group";
    const int nconv = (int)c.conv_dims.size();
    require(c.hidden > 0 && c.n_layers > 0 && c.n_heads > 0 && c.ff > 0, "voicedetect: incomplete wav2vec2 config");
    require(nconv >= 1 && (int)c.conv_kernels.size() == nconv && (int)c.conv_strides.size() == nconv,
            "voicedetect: wav2vec2 conv_dims / conv_kernels / conv_strides lengths differ");
    require(c.hidden % c.n_heads == 0 && c.hidden / c.n_heads == 64,
            "voicedetect: the attention kernel needs head_dim = hidden / n_heads = 64");
    require(layer_fe || group_fe, "voicedetect: feat_extract_norm must be 'group' or 'layer'");
    require(c.feat_extract_activation == "gelu" && c.hidden_act == "gelu",
            "voicedetect: only the gelu activation is supported");
    require(c.pos_k > 0 && c.pos_groups > 0 && c.hidden % c.pos_groups == 0 && (c.hidden / c.pos_groups) % 16 == 0,
            "voicedetect: positional conv groups must split hidden into multiples of 16 channels");
    require(c.pos_norm_dim == 2, "voicedetect: positional conv weight norm must be over dim 2");
    require(c.hidden % 64 == 0 && c.ff % 64 == 0, "voicedetect: hidden and ff_dim must be multiples of 64");
    for (int i = 0; i < nconv; ++i)
        require(c.conv_dims[i] % 64 == 0 && c.conv_kernels[i] >= 1 && c.conv_strides[i] >= 1,
                "voicedetect: wav2vec2 conv layer " + std::to_string(i) + " has an unsupported shape");

    auto f32 = [&](const std::string& name, size_t expect) {
        std::vector<float> v = g.to_f32(name);
        require(v.size() == expect, "voicedetect: tensor '" + name + "' has " + std::to_string(v.size()) +
                                        " values, expected " + std::to_string(expect));
        return v;
    };
    auto norm = [&](const std::string& p, int n, W2Norm& dst) {
        arena.put(f32(p + ".weight", n), &dst.g);
        arena.put(f32(p + ".bias", n), &dst.b);
    };
    // torch [OC][IC][K] (or [OC][IC] for K = 1) -> f16 [OC][K][IC]
    auto conv_w = [&](const std::string& name, int oc, int ic, int k, Layer& l) {
        const std::vector<float> w = f32(name, (size_t)oc * ic * k);
        std::vector<uint16_t> packed((size_t)oc * k * ic);
        for (int o = 0; o < oc; ++o)
            for (int i = 0; i < ic; ++i)
                for (int kk = 0; kk < k; ++kk)
                    packed[((size_t)o * k + kk) * ic + i] = float_to_half_bits(w[((size_t)o * ic + i) * k + kk]);
        l.oc = oc; l.ic = ic; l.k = k;
        arena.put(packed, &l.w);
    };
    auto linear = [&](const std::string& p, int out, int in, Layer& l) {
        conv_w(p + ".weight", out, in, 1, l);
        arena.put(f32(p + ".bias", out), &l.b);
    };

    // conv feature encoder (src/analyze_w2v2.cpp:52-131)
    const int C0 = c.conv_dims[0], K0 = c.conv_kernels[0];
    require(C0 == 256 || C0 == 512 || C0 == 1024, "voicedetect: conv layer 0 must have 256, 512 or 1024 channels");
    require(K0 <= 16 && c.conv_strides[0] <= 8, "voicedetect: conv layer 0 kernel <= 16, stride <= 8");
    const std::string fe = "w2v2.feature_extractor.conv_layers.";
    arena.put(f32(fe + "0.conv.weight", (size_t)C0 * K0), &m.conv0_w);
    if (c.conv_bias) arena.put(f32(fe + "0.conv.bias", C0), &m.conv0_b);
    norm(fe + "0.layer_norm", C0, m.conv0_n);
    m.convs.assign(nconv - 1, Layer());
    m.conv_n.assign(nconv - 1, W2Norm());
    for (int i = 1; i < nconv; ++i) {
        const std::string p = fe + std::to_string(i);
        Layer& l = m.convs[i - 1];
        conv_w(p + ".conv.weight", c.conv_dims[i], c.conv_dims[i - 1], c.conv_kernels[i], l);
        if (c.conv_bias) arena.put(f32(p + ".conv.bias", c.conv_dims[i]), &l.b);
        if (layer_fe) norm(p + ".layer_norm", c.conv_dims[i], m.conv_n[i - 1]);
    }
    const int Cf = c.conv_dims.back(), H = c.hidden;

    // feature projection
    norm("w2v2.feature_projection.layer_norm", Cf, m.fp_n);
    linear("w2v2.feature_projection.projection", H, Cf, m.proj);

    // positional conv: w = g[k] v / ||v[:, :, k]|| (src/analyze_w2v2.cpp:333-359), per group
    {
        const int K = c.pos_k, icg = H / c.pos_groups;
        const std::vector<float> gv = f32("w2v2.encoder.pos_conv_embed.conv.weight_g", (size_t)K);
        const std::vector<float> v = f32("w2v2.encoder.pos_conv_embed.conv.weight_v", (size_t)H * icg * K);
        std::vector<double> sumsq(K, 0.0);
        for (size_t i = 0; i < v.size(); ++i) sumsq[i % K] += (double)v[i] * v[i];
        std::vector<double> sc(K);
        for (int k = 0; k < K; ++k) {
            const double nrm = std::sqrt(sumsq[k]);
            sc[k] = nrm > 0.0 ? (double)gv[k] / nrm : 0.0;
        }
        auto wn = [&](int gi, int o, int i, int k) {
            const size_t src = ((size_t)(gi * icg + o) * icg + i) * K + k;
            return float_to_half_bits((float)((double)v[src] * sc[k]));
        };
        m.pos_fused = (icg == 48 || icg == 64) && K <= 128;
        if (m.pos_fused) {
            // vdk_pos_conv layout [G][64][K][icg], outputs padded to 64 with zeros
            std::vector<uint16_t> packed((size_t)c.pos_groups * 64 * K * icg, 0);
            for (int gi = 0; gi < c.pos_groups; ++gi)
                for (int o = 0; o < icg; ++o)
                    for (int k = 0; k < K; ++k)
                        for (int i = 0; i < icg; ++i)
                            packed[(((size_t)gi * 64 + o) * K + k) * icg + i] = wn(gi, o, i, k);
            m.pos_w.assign(1, nullptr);
            arena.put(packed, &m.pos_w[0]);
        } else {
            // one implicit-GEMM launch per group: input channels padded to a
            // multiple of 32 with zero weights (the GEMM's channel chunk), so
            // group g reads channels g*icg .. g*icg + icp of the projection
            const int icp = (icg + 31) / 32 * 32;
            m.pos_icp = icp;
            m.pos_w.assign(c.pos_groups, nullptr);
            for (int gi = 0; gi < c.pos_groups; ++gi) {
                std::vector<uint16_t> packed((size_t)icg * K * icp, 0);
                for (int o = 0; o < icg; ++o)
                    for (int i = 0; i < icg; ++i)
                        for (int k = 0; k < K; ++k) packed[((size_t)o * K + k) * icp + i] = wn(gi, o, i, k);
                arena.put(packed, &m.pos_w[gi]);
            }
        }
        arena.put(f32("w2v2.encoder.pos_conv_embed.conv.bias", H), &m.pos_b);
    }
    norm("w2v2.encoder.layer_norm", H, m.enc_n);

    // transformer layers; q, k, v stacked into one [3H][H] weight
    m.layers.assign(c.n_layers, W2Layer());
    for (int li = 0; li < c.n_layers; ++li) {
        const std::string p = "w2v2.encoder.layers." + std::to_string(li);
        W2Layer& L = m.layers[li];
        std::vector<uint16_t> wq((size_t)3 * H * H);
        std::vector<float> bq((size_t)3 * H);
        const char* names[3] = {".attention.q_proj", ".attention.k_proj", ".attention.v_proj"};
        for (int j = 0; j < 3; ++j) {
            const std::vector<float> w = f32(p + names[j] + ".weight", (size_t)H * H);
            const std::vector<float> b = f32(p + names[j] + ".bias", (size_t)H);
            for (size_t i = 0; i < w.size(); ++i) wq[(size_t)j * H * H + i] = float_to_half_bits(w[i]);
            std::copy(b.begin(), b.end(), bq.begin() + (size_t)j * H);
        }
        L.qkv.oc = 3 * H; L.qkv.ic = H; L.qkv.k = 1;
        arena.put(wq, &L.qkv.w);
        arena.put(bq, &L.qkv.b);
        linear(p + ".attention.out_proj", H, H, L.out);
        norm(p + ".layer_norm", H, L.ln1);
        linear(p + ".feed_forward.intermediate_dense", c.ff, H, L.ff1);
        linear(p + ".feed_forward.output_dense", H, c.ff, L.ff2);
        norm(p + ".final_layer_norm", H, L.ln2);
    }

    // heads
    const int n_states = c.n_layers + 1;
    m.state_w.assign(n_states, 0.0f);
    if (age_gender) {
        const int ng = (int)cfg_.gender_labels.size();
        require(ng > 0, "voicedetect: age/gender model without gender labels");
        arena.put(f32("age.dense.weight", (size_t)H * H), &m.age_w1);
        arena.put(f32("age.dense.bias", H), &m.age_b1);
        arena.put(f32("age.out_proj.weight", (size_t)H), &m.age_w2);
        arena.put(f32("age.out_proj.bias", 1), &m.age_b2);
        arena.put(f32("gender.dense.weight", (size_t)H * H), &m.gen_w1);
        arena.put(f32("gender.dense.bias", H), &m.gen_b1);
        arena.put(f32("gender.out_proj.weight", (size_t)ng * H), &m.gen_w2);
        arena.put(f32("gender.out_proj.bias", ng), &m.gen_b2);
        m.n_out = 1 + ng;
        m.state_w.back() = 1.0f;   // the heads pool the last hidden state
    } else {
        const int ne = (int)cfg_.emotion_labels.size(), P = c.proj;
        require(ne > 0 && P > 0, "voicedetect: emotion model without labels or classifier_proj_size");
        arena.put(f32("projector.weight", (size_t)P * H), &m.head_w1);
        arena.put(f32("projector.bias", P), &m.head_b1);
        arena.put(f32("classifier.weight", (size_t)ne * P), &m.head_w2);
        arena.put(f32("classifier.bias", ne), &m.head_b2);
        m.n_out = ne;
        // softmax(layer_weights), max-shifted, in double (src/analyze_w2v2.cpp:511-521);
        // without the weighted sum the head reads the last state
        const GgufTensor* lt = g.tensor("layer_weights");
        if (c.weighted_layer_sum && lt && lt->nelements() == n_states) {
            const std::vector<float> lw = g.to_f32("layer_weights");
            double mx = lw[0];
            for (float v : lw) mx = std::max(mx, (double)v);
            double s = 0.0;
            for (int i = 0; i < n_states; ++i) {
                m.state_w[i] = (float)std::exp((double)lw[i] - mx);
                s += m.state_w[i];
            }
            for (float& v : m.state_w) v = (float)(v / s);
        } else {
            m.state_w.back() = 1.0f;
        }
    }
    arena_ = arena.upload();
}

void Model::alloc_w2v2_workspace(int batch, int n) {
    const W2v2Cfg& c = cfg_.w2v2;
    Workspace& w = ws_;
    const int nconv = (int)c.conv_dims.size();
    const int H = c.hidden;
    std::vector<int> T(nconv);
    int t = n;
    for (int i = 0; i < nconv; ++i) {
        t = (t - c.conv_kernels[i]) / c.conv_strides[i] + 1;
        T[i] = t;
    }
    size_t fe_max = 0, fe32_max = 0;
    for (int i = 0; i < nconv; ++i) {
        fe_max = std::max(fe_max, (size_t)batch * T[i] * c.conv_dims[i]);
        if (i > 0 && c.feat_extract_norm == "layer") fe32_max = std::max(fe32_max, (size_t)batch * T[i] * c.conv_dims[i]);
    }
    const size_t BT = (size_t)batch * T.back();
    w.wstats = static_cast<float*>(ws_alloc(sizeof(float) * 2 * batch));
    w.c0_work_bytes = vdk_w2v2_conv0_workspace_size(batch, n, c.conv_dims[0], c.conv_kernels[0], c.conv_strides[0]);
    w.c0_work = ws_alloc(w.c0_work_bytes);
    w.fe[0] = ws_alloc(2 * fe_max);
    w.fe[1] = ws_alloc(2 * fe_max);
    if (fe32_max) w.fe32 = static_cast<float*>(ws_alloc(4 * fe32_max));
    w.u = ws_alloc(2 * BT * c.conv_dims.back());
    // + a zeroed tail: the last positional-conv group reads up to icp - icg
    // channels past the end of the last row (with zero weights)
    w.wproj = ws_alloc(2 * (BT * H + 64));
    VDK_HIP(hipMemsetAsync(w.wproj, 0, 2 * (BT * H + 64), stream_));
    w.z = static_cast<float*>(ws_alloc(4 * BT * H));
    w.acc = static_cast<float*>(ws_alloc(4 * BT * H));
    w.wh = ws_alloc(2 * BT * H);
    w.wh1 = ws_alloc(2 * BT * H);
    w.qkv = ws_alloc(2 * BT * 3 * H);
    w.att = ws_alloc(2 * BT * H);
    w.ffb = ws_alloc(2 * BT * c.ff);
    const int wide = std::max(H, c.proj);
    w.wpool = static_cast<float*>(ws_alloc(4 * (size_t)batch * H));
    w.wt1 = static_cast<float*>(ws_alloc(4 * (size_t)batch * wide));
    w.wt2 = static_cast<float*>(ws_alloc(4 * (size_t)batch * std::max(w2_.n_out, 1)));
    w.raw = static_cast<float*>(ws_alloc(4 * (size_t)batch * std::max(w2_.n_out, 1)));
    size_t fcw = vdk_linear_workspace_size(batch, H, wide);
    fcw = std::max(fcw, vdk_linear_workspace_size(batch, wide, std::max(w2_.n_out, 1)));
    fcw = std::max(fcw, vdk_linear_workspace_size(batch, H, 1));
    w.fc_work_bytes = fcw;
    w.fc_work = ws_alloc(fcw);
}

void Model::analyze_forward(const float* d_pcm, int batch, int n, float* d_raw) {
    const W2v2Cfg& c = cfg_.w2v2;
    const W2v2& m = w2_;
    Workspace& w = ws_;
    const int nconv = (int)c.conv_dims.size();
    const int H = c.hidden, T = analyze_frames(n);
    require(T > 0, "voicedetect: clip too short for the wav2vec2 feature encoder");
    const bool layer_fe = c.feat_extract_norm == "layer";
    const float eps = c.eps;
    const int BT = batch * T;

    // one GEMM-shaped layer over a time-major map: x [B][W][x_stride] -> y
    auto gemm = [&](const char* name, const Layer& l, const void* x, int x_stride, int W, int stride, int pad,
                    int out_w, const float* bias, int act, const void* res, int res_stride, int res_f32,
                    int res_after, void* y, int y_stride, int y_f32) {
        vdk_conv_desc d{};
        d.x = x; d.batch = batch; d.H = 1; d.W = W; d.IC = l.ic; d.x_stride = x_stride;
        d.w = l.w; d.OC = l.oc; d.KH = 1; d.KW = l.k;
        d.stride_h = 1; d.stride_w = stride; d.pad_w = pad; d.dil_h = d.dil_w = 1;
        d.bias = bias; d.act = act;
        d.residual = res; d.res_stride = res_stride; d.res_f32 = res_f32; d.res_after_act = res_after;
        d.y = y; d.y_stride = y_stride; d.y_f32 = y_f32; d.out_w = out_w;
        d.tile = -1;
        conv_ex(name, d);
    };
    auto ln = [&](const char* name, const void* x, int rows, int C, const W2Norm& nrm, int flags, void* y,
                  float* acc, float acc_w) {
        const double in_b = (flags & VDK_LN_X_F32) ? 4.0 : 2.0, out_b = (flags & VDK_LN_Y_F32) ? 4.0 : 2.0;
        prof_begin(name, 0.0, (double)rows * C * (in_b + (y ? out_b : 0.0) + (acc ? 8.0 : 0.0)));
        check_rc(vdk_layer_norm(x, rows, C, nrm.g, nrm.b, eps, flags, y, acc, acc_w, stream_));
        prof_end();
    };

    // -- conv feature encoder --------------------------------------------------
    const float* stats = nullptr;
    if (c.do_normalize) {
        prof_begin("w2v2_wave_stats", 0.0, 8.0 * batch * (double)n);
        check_rc(vdk_wave_stats(d_pcm, batch, n, kWaveNormEps, w.wstats, stream_));
        prof_end();
        stats = w.wstats;
    }
    const int C0 = c.conv_dims[0], K0 = c.conv_kernels[0], S0 = c.conv_strides[0];
    int Tc = (n - K0) / S0 + 1;
    prof_begin("w2v2_conv0", 2.0 * K0 * C0 * (double)batch * Tc, 4.0 * batch * (double)n + 2.0 * batch * Tc * C0);
    check_rc(vdk_w2v2_conv0(d_pcm, batch, n, stats, m.conv0_w, m.conv0_b, C0, K0, S0, layer_fe ? 2 : 1,
                            m.conv0_n.g, m.conv0_n.b, layer_fe ? eps : kGroupNormEps, w.c0_work, w.c0_work_bytes,
                            w.fe[0], stream_));
    prof_end();
    int cur = 0;
    for (int i = 1; i < nconv; ++i) {
        const Layer& l = m.convs[i - 1];
        const int To = (Tc - l.k) / c.conv_strides[i] + 1;
        if (layer_fe) {
            gemm("w2v2_fe_conv", l, w.fe[cur], l.ic, Tc, c.conv_strides[i], 0, 0, l.b, VDK_ACT_NONE, nullptr, 0, 0, 0,
                 w.fe32, l.oc, 1);
            ln("w2v2_fe_ln", w.fe32, batch * To, l.oc, m.conv_n[i - 1], VDK_LN_X_F32 | VDK_LN_GELU, w.fe[cur ^ 1],
               nullptr, 0.0f);
        } else {
            gemm("w2v2_fe_conv", l, w.fe[cur], l.ic, Tc, c.conv_strides[i], 0, 0, l.b, VDK_ACT_GELU, nullptr, 0, 0, 0,
                 w.fe[cur ^ 1], l.oc, 0);
        }
        cur ^= 1;
        Tc = To;
    }
    w.feat_buf = cur;
    const int Cf = c.conv_dims.back();

    // -- feature projection + positional conv ----------------------------------
    ln("w2v2_fp_ln", w.fe[cur], BT, Cf, m.fp_n, 0, w.u, nullptr, 0.0f);
    gemm("w2v2_proj", m.proj, w.u, Cf, T, 1, 0, 0, m.proj.b, VDK_ACT_NONE, nullptr, 0, 0, 0, w.wproj, H, 0);
    if (m.pos_fused) {
        prof_begin("w2v2_pos_conv", 2.0 * BT * (double)H * (H / c.pos_groups) * c.pos_k,
                   2.0 * BT * H * 2.0 + 4.0 * BT * H);
        check_rc(vdk_pos_conv(w.wproj, batch, T, H, c.pos_groups, m.pos_w[0], m.pos_b, c.pos_k, c.pos_k / 2, w.z,
                              stream_));
        prof_end();
    } else {
        const int icg = H / c.pos_groups;
        Layer pl;
        pl.ic = m.pos_icp; pl.oc = icg; pl.k = c.pos_k;
        for (int gi = 0; gi < c.pos_groups; ++gi) {
            pl.w = m.pos_w[gi];
            const half_t* xg = static_cast<const half_t*>(w.wproj) + (size_t)gi * icg;
            gemm("w2v2_pos_conv", pl, xg, H, T, 1, c.pos_k / 2, T, m.pos_b + gi * icg, VDK_ACT_GELU, xg, H, 0, 1,
                 w.z + (size_t)gi * icg, H, 1);
        }
    }

    // -- transformer ------------------------------------------------------------
    const float scale = 1.0f / std::sqrt((float)(H / c.n_heads));
    const std::vector<float>& sw = m.state_w;
    const bool emotion = cfg_.arch == "wav2vec2_emotion";
    auto attention = [&](const W2Layer& L, const void* hin, int res_f32, const void* res, void* y, int y_f32) {
        gemm("w2v2_qkv", L.qkv, hin, H, T, 1, 0, 0, L.qkv.b, VDK_ACT_NONE, nullptr, 0, 0, 0, w.qkv, 3 * H, 0);
        prof_begin("w2v2_attention", 4.0 * batch * (double)T * T * H, 2.0 * BT * 4.0 * H);
        check_rc(vdk_attention(w.qkv, batch, T, c.n_heads, H / c.n_heads, scale, w.att, stream_));
        prof_end();
        gemm("w2v2_out", L.out, w.att, H, T, 1, 0, 0, L.out.b, VDK_ACT_NONE, res, H, res_f32, 0, y, H, y_f32);
    };
    auto feed_forward = [&](const W2Layer& L, const void* hin, int res_f32, const void* res, void* y, int y_f32) {
        gemm("w2v2_ff1", L.ff1, hin, H, T, 1, 0, 0, L.ff1.b, VDK_ACT_GELU, nullptr, 0, 0, 0, w.ffb, c.ff, 0);
        gemm("w2v2_ff2", L.ff2, w.ffb, c.ff, T, 1, 0, 0, L.ff2.b, VDK_ACT_NONE, res, H, res_f32, 0, y, H, y_f32);
    };
    // The heads pool sum_i w_i mean_t(hidden_states[i]) (w: softmax(layer_weights)
    // for the emotion head's weighted layer sum, else one-hot on the last state)
    // into wpool, one state at a time.
    bool pooled = false;
    auto pool_state = [&](const void* xs, int x_f32, int i) {
        if (sw[i] == 0.0f) return;
        prof_begin("w2v2_time_mean", 0.0, (x_f32 ? 4.0 : 2.0) * BT * H);
        check_rc(vdk_time_mean_acc(xs, x_f32, batch, T, H, sw[i], pooled ? 1 : 0, w.wpool, stream_));
        prof_end();
        pooled = true;
    };
    if (c.stable_layer_norm) {
        // pre-norm (src/analyze_w2v2.cpp:398-427): w.z is the residual stream r;
        // hidden_states[i] is the input of layer i, the last one the final LN
        for (int li = 0; li < c.n_layers; ++li) {
            const W2Layer& L = m.layers[li];
            pool_state(w.z, 1, li);
            ln("w2v2_ln", w.z, BT, H, L.ln1, VDK_LN_X_F32, w.wh, nullptr, 0.0f);
            attention(L, w.wh, 1, w.z, w.z, 1);
            ln("w2v2_ln", w.z, BT, H, L.ln2, VDK_LN_X_F32, w.wh1, nullptr, 0.0f);
            feed_forward(L, w.wh1, 1, w.z, w.z, 1);
        }
        // the final LN in f32 (the last hidden state; read back by analyze_capture)
        ln("w2v2_ln", w.z, BT, H, m.enc_n, VDK_LN_X_F32 | VDK_LN_Y_F32, w.acc, nullptr, 0.0f);
        pool_state(w.acc, 1, c.n_layers);
    } else {
        // post-norm (src/analyze_w2v2.cpp:429-468): hidden_states[0] is the
        // encoder LN of (projection + pos conv), then every layer's output
        ln("w2v2_ln", w.z, BT, H, m.enc_n, VDK_LN_X_F32, w.wh, nullptr, 0.0f);
        pool_state(w.wh, 0, 0);
        for (int li = 0; li < c.n_layers; ++li) {
            const W2Layer& L = m.layers[li];
            attention(L, w.wh, 0, w.wh, w.z, 1);
            ln("w2v2_ln", w.z, BT, H, L.ln1, VDK_LN_X_F32, w.wh1, nullptr, 0.0f);
            feed_forward(L, w.wh1, 0, w.wh1, w.z, 1);
            ln("w2v2_ln", w.z, BT, H, L.ln2, VDK_LN_X_F32, w.wh, nullptr, 0.0f);
            pool_state(w.wh, 0, li + 1);
        }
    }
    require(pooled, "voicedetect: the analyze head pools no hidden state");

    // -- heads ------------------------------------------------------------------
    if (emotion) {
        const int P = c.proj, ne = m.n_out;
        linear("w2v2_projector", w.wpool, batch, H, m.head_w1, m.head_b1, nullptr, P, 0, w.wt1);
        linear("w2v2_classifier", w.wt1, batch, P, m.head_w2, m.head_b2, nullptr, ne, 0, d_raw);
    } else {
        const int ng = m.n_out - 1;
        auto head = [&](const char* n1, const char* n2, const float* w1, const float* b1, const float* w2,
                        const float* b2, int n_out, float* out) {
            prof_begin(n1, 2.0 * batch * (double)H * H, 4.0 * (double)H * H);
            check_rc(vdk_linear_ex(w.wpool, batch, H, w1, b1, nullptr, H, VDK_ACT_TANH, w.wt1, w.fc_work,
                                   w.fc_work_bytes, stream_));
            prof_end();
            linear(n2, w.wt1, batch, H, w2, b2, nullptr, n_out, 0, out);
        };
        head("w2v2_age_dense", "w2v2_age_out", m.age_w1, m.age_b1, m.age_w2, m.age_b2, 1, w.wt2);
        VDK_HIP(hipMemcpy2DAsync(d_raw, sizeof(float) * m.n_out, w.wt2, sizeof(float), sizeof(float), batch,
                                 hipMemcpyDeviceToDevice, stream_));
        head("w2v2_gender_dense", "w2v2_gender_out", m.gen_w1, m.gen_b1, m.gen_w2, m.gen_b2, ng, w.wt2);
        VDK_HIP(hipMemcpy2DAsync(d_raw + 1, sizeof(float) * m.n_out, w.wt2, sizeof(float) * ng, sizeof(float) * ng,
                                 batch, hipMemcpyDeviceToDevice, stream_));
    }
}

void Model::analyze_batch_device(const float* d_pcm, int batch, int n, float* d_raw) {
    std::lock_guard<std::mutex> lock(mu_);
    require(is_analyzer(), "voicedetect: this model has no age/gender/emotion analyze heads");
    require(batch > 0 && d_pcm && d_raw, "voicedetect: invalid analyze batch");
    require(analyze_frames(n) > 0, "voicedetect: clip too short for the wav2vec2 feature encoder");
    ensure_device();
    ensure_workspace(batch, n);
    analyze_forward(d_pcm, batch, n, d_raw);
}

void Model::analyze_capture(const float* pcm, int batch, int n, float* feat, float* hidden, float* raw) {
    std::lock_guard<std::mutex> lock(mu_);
    require(is_analyzer(), "voicedetect: this model has no age/gender/emotion analyze heads");
    require(batch > 0 && pcm, "voicedetect: invalid analyze batch");
    const int T = analyze_frames(n);
    require(T > 0, "voicedetect: clip too short for the wav2vec2 feature encoder");
    ensure_device();
    ensure_workspace(batch, n);
    const W2v2Cfg& c = cfg_.w2v2;
    VDK_HIP(hipMemcpyAsync(ws_.pcm, pcm, sizeof(float) * (size_t)batch * n, hipMemcpyHostToDevice, stream_));
    analyze_forward(ws_.pcm, batch, n, ws_.raw);
    const size_t BT = (size_t)batch * T;
    std::vector<uint16_t> h16;
    auto widen = [&](const void* src, size_t count, float* dst) {
        h16.resize(count);
        VDK_HIP(hipMemcpyAsync(h16.data(), src, 2 * count, hipMemcpyDeviceToHost, stream_));
        VDK_HIP(hipStreamSynchronize(stream_));
        for (size_t i = 0; i < count; ++i) dst[i] = half_bits_to_float(h16[i]);
    };
    if (feat) widen(ws_.fe[ws_.feat_buf], BT * c.conv_dims.back(), feat);
    if (hidden) {
        // the last hidden state: the final LN output (f32) for the pre-norm
        // stack, the last layer's f16 LN output for the post-norm one
        if (c.stable_layer_norm)
            VDK_HIP(hipMemcpyAsync(hidden, ws_.acc, 4 * BT * c.hidden, hipMemcpyDeviceToHost, stream_));
        else
            widen(ws_.wh, BT * c.hidden, hidden);
    }
    if (raw) VDK_HIP(hipMemcpyAsync(raw, ws_.raw, 4 * (size_t)batch * w2_.n_out, hipMemcpyDeviceToHost, stream_));
    VDK_HIP(hipStreamSynchronize(stream_));
}

void Model::analyze_batch_host(const float* pcm, int batch, int n, float* raw) {
    analyze_capture(pcm, batch, n, nullptr, nullptr, raw);
}

std::string Model::analyze_json(const std::vector<float>& pcm, int sample_rate) {
    const std::vector<float> x = sample_rate == 16000 ? pcm : resample_linear(pcm, sample_rate, 16000);
    std::vector<float> raw((size_t)analyze_outputs());
    analyze_batch_host(x.data(), 1, (int)x.size(), raw.data());
    const bool ag = cfg_.arch == "wav2vec2_age_gender";
    const std::vector<std::string>& labels = ag ? cfg_.gender_labels : cfg_.emotion_labels;
    // softmax over the logits, argmax (first maximum) -> label
    // (src/analyze_w2v2.cpp:566-578, 640-652)
    std::vector<float> logits(raw.begin() + (ag && !raw.empty() ? 1 : 0), raw.end());
    std::vector<float> probs(logits.size());
    int am = 0;
    if (!logits.empty()) {
        double mx = logits[0];
        for (float v : logits) mx = std::max(mx, (double)v);
        double s = 0.0;
        for (size_t i = 0; i < logits.size(); ++i) {
            probs[i] = (float)std::exp((double)logits[i] - mx);
            s += probs[i];
        }
        for (float& v : probs) v = (float)(v / s);
        for (size_t i = 1; i < logits.size(); ++i)
            if (logits[i] > logits[am]) am = (int)i;
    }
    const std::string dom = am < (int)labels.size() ? labels[am] : "";
    auto num = [](double v) {
        char buf[32];
        std::snprintf(buf, sizeof(buf), "%.6g", v);
        return std::string(buf);
    };
    std::string js;
    if (ag) {
        const double age = raw.empty() ? 0.0 : (double)raw[0] * 100.0;
        js = "{\"age\":" + num(age) + ",\"gender\":{\"label\":\"" + dom + "\"";
        for (size_t i = 0; i < labels.size(); ++i)
            js += ",\"" + labels[i] + "\":" + num(i < probs.size() ? probs[i] : 0.0f);
        js += "}}";
    } else {
        js = "{\"emotion\":{\"label\":\"" + dom + "\",\"scores\":{";
        for (size_t i = 0; i < labels.size(); ++i) {
            if (i) js += ",";
            js += "\"" + labels[i] + "\":" + num(i < probs.size() ? probs[i] : 0.0f);
        }
        js += "}}}";
    }
    return js;
}

}  // namespace vdk
