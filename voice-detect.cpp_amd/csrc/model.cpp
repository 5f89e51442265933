// model.cpp - see model.hpp.
#include "model.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>

#include "arena.hpp"
#include "audio.hpp"
#include "common.hpp"

namespace vdk {

void check_rc(int rc) {
    if (rc != 0) throw Error(vdk_last_error());
}

namespace {
void check(int rc) { check_rc(rc); }
}  // namespace

std::unique_ptr<Model> Model::load(const std::string& path) {
    std::unique_ptr<Model> m(new Model());
    m->gguf_.reset(new GgufFile(path));
    const GgufFile& g = *m->gguf_;
    ModelConfig& c = m->cfg_;
    // src/model_loader.cpp:114-133
    c.arch = g.str("voicedetect.arch");
    c.embedding_dim = (int)g.u32("voicedetect.embedding_dim", 0);
    c.l2_normalize = g.boolean("voicedetect.l2_normalize", true);
    c.fbank.sample_rate = (int)g.u32("voicedetect.fbank.sample_rate", 16000);
    c.fbank.n_mels = (int)g.u32("voicedetect.fbank.n_mels", 80);
    c.fbank.n_fft = (int)g.u32("voicedetect.fbank.n_fft", 512);
    c.fbank.win_length = (int)g.u32("voicedetect.fbank.win_length", 400);
    c.fbank.hop_length = (int)g.u32("voicedetect.fbank.hop_length", 160);
    c.fbank.preemph = g.f32("voicedetect.fbank.preemph", 0.97f);
    c.fbank.low_freq = g.f32("voicedetect.fbank.low_freq", 20.0f);
    c.fbank.high_freq = g.f32("voicedetect.fbank.high_freq", 0.0f);
    c.fbank.cmn = g.boolean("voicedetect.fbank.cmn", true) ? 1 : 0;
    c.analyze_present = g.boolean("voicedetect.analyze.present", false);
    if (c.arch == "wespeaker_resnet34") {
        ResNetCfg& r = c.resnet;   // src/model_loader.cpp:135-150
        const std::string p = "voicedetect.resnet.";
        r.stem_weight = g.str(p + "stem_weight");
        r.stem_bias = g.str(p + "stem_bias");
        r.conv1_weight = g.str_arr(p + "conv1_weight");
        r.conv1_bias = g.str_arr(p + "conv1_bias");
        r.conv2_weight = g.str_arr(p + "conv2_weight");
        r.conv2_bias = g.str_arr(p + "conv2_bias");
        r.down_weight = g.str_arr(p + "down_weight");
        r.down_bias = g.str_arr(p + "down_bias");
        r.stride = g.i32_arr(p + "stride");
        r.seg_weight = g.str(p + "seg_weight");
        r.seg_bias = g.str(p + "seg_bias");
        r.mean_vec = g.str(p + "mean_vec");
        r.var_eps = g.f32(p + "var_eps", 1e-8f);
    }
    if (c.arch == "eres2net") {
        ERes2NetCfg& e = c.eres2net;   // src/model_loader.cpp:151-163
        const std::string p = "voicedetect.eres2net.";
        e.conv_weight = g.str_arr(p + "conv_weight");
        e.conv_bias = g.str_arr(p + "conv_bias");
        e.conv_stride = g.i32_arr(p + "conv_stride");
        e.num_blocks = g.i32_arr(p + "num_blocks");
        e.m_channels = (int)g.u32(p + "m_channels", 0);
        e.scale = (int)g.u32(p + "scale", 2);
        e.seg_weight = g.str(p + "seg_weight");
        e.seg_bias = g.str(p + "seg_bias");
        e.relu_clamp = g.f32(p + "relu_clamp", 20.0f);
        e.var_eps = g.f32(p + "var_eps", 1e-8f);
    }
    if (c.arch == "campplus") {
        CamPPlusCfg& cp = c.campplus;   // src/model_loader.cpp:165-173
        const std::string p = "voicedetect.campplus.";
        cp.conv_weight = g.str_arr(p + "conv_weight");
        cp.conv_bias = g.str_arr(p + "conv_bias");
        cp.bn_prefix = g.str_arr(p + "bn_prefix");
        cp.emb_bn_mean = g.str(p + "emb_bn_mean");
        cp.emb_bn_var = g.str(p + "emb_bn_var");
        cp.bn_eps = g.f32(p + "bn_eps", 1e-5f);
    }
    if (c.analyze_present) {   // src/model_loader.cpp:175-180
        c.emotion_labels = g.str_arr("voicedetect.analyze.emotion_labels");
        c.gender_labels = g.str_arr("voicedetect.analyze.gender_labels");
    }
    if (c.arch == "wav2vec2_emotion" || c.arch == "wav2vec2_age_gender") {
        W2v2Cfg& w = c.w2v2;   // src/model_loader.cpp:181-207
        const std::string p = "voicedetect.w2v2.";
        w.hidden = (int)g.u32(p + "hidden_size", 0);
        w.n_layers = (int)g.u32(p + "n_layers", 0);
        w.n_heads = (int)g.u32(p + "n_heads", 0);
        w.ff = (int)g.u32(p + "ff_dim", 0);
        w.conv_dims = g.i32_arr(p + "conv_dims");
        w.conv_kernels = g.i32_arr(p + "conv_kernels");
        w.conv_strides = g.i32_arr(p + "conv_strides");
        w.feat_extract_norm = g.str(p + "feat_extract_norm");
        w.conv_bias = g.boolean(p + "conv_bias", false);
        w.do_normalize = g.boolean(p + "do_normalize", false);
        w.feat_extract_activation = g.str(p + "feat_extract_activation");
        w.hidden_act = g.str(p + "hidden_act");
        w.stable_layer_norm = g.boolean(p + "do_stable_layer_norm", false);
        w.eps = g.f32(p + "layer_norm_eps", 1e-5f);
        w.pos_k = (int)g.u32(p + "num_conv_pos_embeddings", 0);
        w.pos_groups = (int)g.u32(p + "num_conv_pos_embedding_groups", 0);
        w.pos_norm_dim = (int)g.u32(p + "pos_conv_weight_norm_dim", 2);
        w.weighted_layer_sum = g.boolean(p + "use_weighted_layer_sum", false);
        w.proj = (int)g.u32(p + "classifier_proj_size", 0);
    }
    // src/model_loader.cpp:212-214: a speaker model needs an embedding dim.
    if (c.embedding_dim <= 0 && !c.analyze_present) throw Error("gguf: voicedetect.embedding_dim missing");
    return m;
}

Model::~Model() {
    free_workspace();
    for (hipEvent_t e : event_pool_) (void)hipEventDestroy(e);
    for (auto& p : pending_) { (void)hipEventDestroy(p.a); (void)hipEventDestroy(p.b); }
    if (arena_) (void)hipFree(arena_);
    if (fb_tables_) (void)hipFree(fb_tables_);
    if (prof_marker_) (void)hipFree(prof_marker_);
    if (stream_) (void)hipStreamDestroy(stream_);
}

int Model::frames(int n_samples) const {
    const vdk_fbank_cfg& f = cfg_.fbank;
    if (n_samples < f.win_length || f.hop_length <= 0) return 0;
    return 1 + (n_samples - f.win_length) / f.hop_length;
}

// ECAPA pads every conv by reflection without repeating the edge frame
// (src/encoder.cpp:32-52), which needs pad < T; the reference builds
// out-of-range row indices below that and SpeechBrain's reflect pad raises.
// The widest pad is max((k0 - 1) / 2, the last SE-Res2Net block's dilation).
int Model::min_frames() const {
    if (cfg_.arch != "ecapa_tdnn") return 1;
    int pad = 0;
    if (const GgufTensor* t = gguf_->tensor("blocks.0.conv.conv.weight"))
        if (t->ne.size() == 3) pad = (int)(t->ne[0] - 1) / 2;
    int n_res = 0;
    while (gguf_->tensor("blocks." + std::to_string(n_res + 1) + ".tdnn1.conv.conv.weight")) ++n_res;
    if (n_res > 0) pad = std::max(pad, n_res + 1);
    return pad + 1;
}

void Model::check_frames(int n_samples) const {
    const int T = frames(n_samples);
    if (T <= 0) throw Error("voicedetect: FBank produced no frames");
    const int need = min_frames();
    if (T < need)
        throw Error("voicedetect: clip too short for reflect padding (" + std::to_string(T) + " frames, the model needs " +
                    std::to_string(need) + ")");
}

void Model::ensure_device() {
    if (ready_) return;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) throw Error("voicedetect: no HIP device available");
    VDK_HIP(hipGetDevice(&device_));
    const bool resnet = cfg_.arch == "wespeaker_resnet34", ecapa = cfg_.arch == "ecapa_tdnn";
    const bool campp = cfg_.arch == "campplus", eres = cfg_.arch == "eres2net";
    if (!resnet && !ecapa && !campp && !eres && !is_analyzer())
        throw Error("voicedetect: unsupported arch '" + cfg_.arch + "'");
    if (!stream_) VDK_HIP(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
    if (is_analyzer()) {   // raw-waveform model: no FBank front end
        upload_w2v2();
        ready_ = true;
        return;
    }
    const size_t tb = vdk_fbank_tables_size(&cfg_.fbank);
    if (tb == 0) throw Error(vdk_last_error());
    if (!fb_tables_) VDK_HIP(hipMalloc(&fb_tables_, tb));
    check(vdk_fbank_tables_fill(&cfg_.fbank, fb_tables_));
    if (resnet) upload_resnet();
    else if (ecapa) upload_ecapa();
    else if (campp) upload_campplus();
    else upload_eres2net();
    ready_ = true;
}

void Model::upload_resnet() {
    const GgufFile& g = *gguf_;
    const ResNetCfg& r = cfg_.resnet;
    const size_t nb = r.conv1_weight.size();
    require(nb > 0 && r.conv1_bias.size() == nb && r.conv2_weight.size() == nb && r.conv2_bias.size() == nb &&
                r.down_weight.size() == nb && r.down_bias.size() == nb && r.stride.size() == nb,
            "voicedetect: inconsistent resnet block manifest");
    ArenaBuilder arena;
    auto put_f32 = [&](const std::string& name, size_t expect, float** dst) {
        std::vector<float> v = g.to_f32(name);
        require(expect == 0 || v.size() == expect, "voicedetect: tensor '" + name + "' has the wrong size");
        arena.put(v, dst);
        return v.size();
    };
    // conv weight ne = [KW, KH, IC, OC] -> f16 [OC][KH][KW][IC]
    auto put_conv = [&](const std::string& wn, const std::string& bn, int ic, int k, int stride, int pad,
                        Conv& c) {
        const GgufTensor* t = g.tensor(wn);
        require(t != nullptr, "voicedetect: missing tensor '" + wn + "'");
        require(t->ne.size() == 4 && t->ne[0] == k && t->ne[1] == k && t->ne[2] == ic,
                "voicedetect: conv weight '" + wn + "' has an unexpected shape");
        const int oc = (int)t->ne[3];
        require(oc % 32 == 0 && ic % 16 == 0,
                "voicedetect: conv '" + wn + "' needs IC % 16 == 0 and OC % 32 == 0");
        std::vector<uint16_t> packed((size_t)oc * k * k * ic);
        const uint16_t* h16 = t->type == GGML_F16 ? reinterpret_cast<const uint16_t*>(t->data) : nullptr;
        std::vector<float> f32;
        if (!h16) f32 = g.to_f32(wn);
        for (int o = 0; o < oc; ++o)
            for (int i = 0; i < ic; ++i)
                for (int kh = 0; kh < k; ++kh)
                    for (int kw = 0; kw < k; ++kw) {
                        const size_t src = (((size_t)o * ic + i) * k + kh) * k + kw;
                        const size_t dst = (((size_t)o * k + kh) * k + kw) * ic + i;
                        packed[dst] = h16 ? h16[src] : float_to_half_bits(f32[src]);
                    }
        c.ic = ic; c.oc = oc; c.k = k; c.stride = stride; c.pad = pad;
        arena.put(packed, &c.w);
        // the band kernels stream whole-line weight chunks; the register-weight
        // kernels load their A fragments from it as whole kilobytes
        if (k == 3 && stride == 1 && ic % 16 == 0 && (oc % 128 == 0 || oc == 32 || oc == 64)) {
            std::vector<uint16_t> chunked(packed.size());
            vdk_conv_pack_chunked(packed.data(), oc, k, k, ic, chunked.data());
            arena.put(chunked, &c.wc);
        }
        put_f32(bn, (size_t)oc, &c.b);
        return oc;
    };

    // stem: ne [3, 3, 1, OC], f32 on the device (the stem runs in f32)
    const GgufTensor* st = g.tensor(r.stem_weight);
    require(st && st->ne.size() == 4 && st->ne[0] == 3 && st->ne[1] == 3 && st->ne[2] == 1,
            "voicedetect: stem weight must be [3,3,1,OC]");
    stem_oc_ = (int)st->ne[3];
    require(stem_oc_ == 16 || stem_oc_ == 32 || stem_oc_ == 64, "voicedetect: stem OC must be 16, 32 or 64");
    put_f32(r.stem_weight, (size_t)stem_oc_ * 9, &stem_w_);
    put_f32(r.stem_bias, (size_t)stem_oc_, &stem_b_);
    blocks_.assign(nb, Block());
    int C = stem_oc_, H = cfg_.fbank.n_mels;
    for (size_t i = 0; i < nb; ++i) {
        Block& b = blocks_[i];
        const int s = r.stride[i];
        require(s == 1 || s == 2, "voicedetect: block stride must be 1 or 2");
        const int oc = put_conv(r.conv1_weight[i], r.conv1_bias[i], C, 3, s, 1, b.c1);
        put_conv(r.conv2_weight[i], r.conv2_bias[i], oc, 3, 1, 1, b.c2);
        require(b.c2.oc == oc, "voicedetect: conv2 width differs from conv1");
        b.has_down = !r.down_weight[i].empty();
        if (b.has_down) {
            put_conv(r.down_weight[i], r.down_bias[i], C, 1, s, 0, b.down);
            require(b.down.oc == oc, "voicedetect: downsample width differs from conv1");
        } else {
            require(s == 1 && C == oc, "voicedetect: identity shortcut needs stride 1 and equal widths");
        }
        C = oc;
        H = (H - 1) / s + 1;
    }
    pooled_dim_ = 2 * C * H;
    const size_t nseg = put_f32(r.seg_weight, 0, &seg_w_);
    require(nseg == (size_t)pooled_dim_ * cfg_.embedding_dim,
            "voicedetect: seg weight must be [embedding_dim, 2*C*H']");
    if (!r.seg_bias.empty()) put_f32(r.seg_bias, (size_t)cfg_.embedding_dim, &seg_b_);
    if (!r.mean_vec.empty()) put_f32(r.mean_vec, (size_t)cfg_.embedding_dim, &mean_vec_);

    arena_ = arena.upload();
}

void* Model::ws_alloc(size_t bytes) {
    void* p = nullptr;
    VDK_HIP(hipMalloc(&p, bytes < 256 ? 256 : bytes));
    ws_.allocs.push_back(p);
    return p;
}

void Model::free_workspace() {
    for (void* p : ws_.allocs) (void)hipFree(p);
    ws_ = Workspace();
}

void Model::ensure_workspace(int batch, int n_samples) {
    if (!ws_.allocs.empty() && batch <= ws_.batch && n_samples == ws_.n_samples) return;
    VDK_HIP(hipStreamSynchronize(stream_));
    free_workspace();
    const int T = frames(n_samples);
    const int nmel = cfg_.fbank.n_mels;
    Workspace& w = ws_;
    w.batch = batch;
    w.n_samples = n_samples;
    w.pcm = static_cast<float*>(ws_alloc(sizeof(float) * (size_t)batch * n_samples));
    if (is_analyzer()) {
        alloc_w2v2_workspace(batch, n_samples);
        return;
    }
    w.feats = static_cast<float*>(ws_alloc(sizeof(float) * (size_t)batch * nmel * T));
    if (cfg_.fbank.cmn) {
        w.fb_mean = static_cast<float*>(ws_alloc(sizeof(float) * (size_t)batch * nmel));
        w.fb_work_bytes = vdk_fbank_workspace_size(&cfg_.fbank, batch, n_samples);
        w.fb_work = ws_alloc(w.fb_work_bytes);
    }
    w.pooled = static_cast<float*>(ws_alloc(sizeof(float) * (size_t)batch * pooled_dim_));
    w.pre = static_cast<float*>(ws_alloc(sizeof(float) * (size_t)batch * cfg_.embedding_dim));
    w.emb = static_cast<float*>(ws_alloc(sizeof(float) * (size_t)batch * cfg_.embedding_dim));
    if (cfg_.arch == "ecapa_tdnn") alloc_ecapa_workspace(batch, T);
    else if (cfg_.arch == "campplus") alloc_campplus_workspace(batch, T);
    else if (cfg_.arch == "eres2net") alloc_eres2net_workspace(batch, T);
    else alloc_resnet_workspace(batch, T);
}

void Model::alloc_resnet_workspace(int batch, int T) {
    const int nmel = cfg_.fbank.n_mels;
    size_t act = (size_t)nmel * T * stem_oc_;
    int H = nmel, W = T;
    for (const Block& b : blocks_) {
        H = (H - 1) / b.c1.stride + 1;
        W = (W - 1) / b.c1.stride + 1;
        act = std::max(act, (size_t)H * W * b.c1.oc);
    }
    Workspace& w = ws_;
    w.act_bytes = act * 2 * batch;
    for (int i = 0; i < 4; ++i) w.act[i] = ws_alloc(w.act_bytes);
    w.fc_work_bytes = vdk_linear_workspace_size(batch, pooled_dim_, cfg_.embedding_dim);
    w.fc_work = ws_alloc(w.fc_work_bytes);
}

void Model::prof_begin(const char* name, double flops, double bytes) {
    prof_open_ = false;
    if (!profiling_) return;
    if (!prof_filter_.empty() && std::strncmp(name, prof_filter_.c_str(), prof_filter_.size()) != 0) return;
    auto ev = [&] {
        hipEvent_t e;
        if (!event_pool_.empty()) { e = event_pool_.back(); event_pool_.pop_back(); }
        // timing-only events: no system-scope fence, so recording one does
        // not write back and invalidate the caches around the kernel it brackets
        // (take_profile synchronizes the stream before reading them)
        else VDK_HIP(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
        return e;
    };
    Pending p{name, flops, bytes, ev(), ev()};
    if (prof_markers_) launch_profile_marker(prof_marker_, 1, stream_);
    VDK_HIP(hipEventRecord(p.a, stream_));
    pending_.push_back(p);
    prof_open_ = true;
}

void Model::prof_end() {
    if (!prof_open_) return;
    VDK_HIP(hipEventRecord(pending_.back().b, stream_));
    if (prof_markers_) launch_profile_marker(prof_marker_, 2, stream_);
    prof_open_ = false;
}

void Model::conv(const Conv& c, const void* x, int batch, int H, int W, const void* res, int relu, void* y) {
    const int Ho = (H + 2 * c.pad - c.k) / c.stride + 1, Wo = (W + 2 * c.pad - c.k) / c.stride + 1;
    if (profiling_) {
        const double npix = (double)batch * Ho * Wo;
        const double flops = 2.0 * c.k * c.k * c.ic * c.oc * npix;
        const double bytes = 2.0 * ((double)batch * H * W * c.ic + (double)c.oc * c.k * c.k * c.ic +
                                    npix * c.oc * (res ? 2.0 : 1.0)) + 4.0 * c.oc;
        std::string name = "conv" + std::to_string(c.k) + "x" + std::to_string(c.k) + "_s" +
                           std::to_string(c.stride) + "_" + std::to_string(c.ic) + "to" + std::to_string(c.oc);
        prof_begin(name.c_str(), flops, bytes);
    }
    vdk_conv_desc d{};
    d.x = x; d.batch = batch; d.H = H; d.W = W; d.IC = c.ic;
    d.w = c.w; d.w_chunked = c.wc; d.OC = c.oc; d.KH = d.KW = c.k;
    d.stride_h = d.stride_w = c.stride;
    d.pad_h = d.pad_w = c.pad;
    d.bias = c.b; d.residual = res; d.act = relu ? VDK_ACT_RELU : VDK_ACT_NONE; d.y = y; d.tile = -1;
    check(vdk_conv2d_ex(&d, stream_));
    prof_end();
}

void Model::forward(const float* d_pcm, int batch, int n_samples, float* d_out) {
    const int T = frames(n_samples);
    if (T <= 0) throw Error("voicedetect: FBank produced no frames");
    const int nmel = cfg_.fbank.n_mels;
    // FBank front end
    prof_begin("fbank", 0.0, 4.0 * batch * ((double)n_samples + (double)nmel * T));
    // the features stay un-normalised: the encoder's first kernel subtracts
    // the CMN means as it loads them
    check(vdk_fbank_ex(&cfg_.fbank, fb_tables_, d_pcm, batch, n_samples, ws_.feats, ws_.fb_mean, ws_.fb_work,
                       ws_.fb_work_bytes, stream_));
    prof_end();
    // with L2 normalisation the encoder's embedding FC writes the normalised
    // rows straight into the output (the pre-norm rows stay in ws_.pre)
    l2_dst_ = cfg_.l2_normalize ? d_out : nullptr;
    if (cfg_.arch == "ecapa_tdnn") encode_ecapa(batch, T);
    else if (cfg_.arch == "campplus") encode_campplus(batch, T);
    else if (cfg_.arch == "eres2net") encode_eres2net(batch, T);
    else encode_resnet(batch, T);
    l2_dst_ = nullptr;
    const int E = cfg_.embedding_dim;
    if (!cfg_.l2_normalize)
        VDK_HIP(hipMemcpyAsync(d_out, ws_.pre, sizeof(float) * (size_t)batch * E, hipMemcpyDeviceToDevice, stream_));
}

void Model::embed_fc(const char* name, const float* x, int batch, int in_dim, const float* w, const float* b,
                     const float* mv, int out_dim) {
    prof_begin(name, 2.0 * batch * (double)in_dim * out_dim,
               4.0 * ((double)batch * in_dim + (double)in_dim * out_dim + 2.0 * batch * out_dim));
    if (l2_dst_)
        check(vdk_linear_l2_ex(x, batch, in_dim, w, b, mv, out_dim, ws_.pre, l2_dst_, ws_.fc_work, ws_.fc_work_bytes,
                               stream_));
    else
        check(vdk_linear_ex(x, batch, in_dim, w, b, mv, out_dim, VDK_ACT_NONE, ws_.pre, ws_.fc_work,
                            ws_.fc_work_bytes, stream_));
    prof_end();
}

void Model::encode_resnet(int batch, int T) {
    const int nmel = cfg_.fbank.n_mels;
    // stem conv + ReLU
    prof_begin("stem3x3", 2.0 * 9 * stem_oc_ * (double)batch * nmel * T,
               4.0 * batch * nmel * T + 2.0 * batch * nmel * T * stem_oc_);
    check(vdk_stem_conv3x3_ex(ws_.feats, ws_.fb_mean, batch, nmel, T, stem_w_, stem_b_, stem_oc_, 1, 0, ws_.act[0],
                              stream_));
    prof_end();
    int xi = 0, C = stem_oc_, H = nmel, W = T;
    for (const Block& b : blocks_) {
        int others[3], k = 0;
        for (int i = 0; i < 4; ++i)
            if (i != xi) others[k++] = i;
        void* x = ws_.act[xi];
        void* h = ws_.act[others[0]];
        void* d = ws_.act[others[1]];
        void* y = ws_.act[others[2]];
        const int s = b.c1.stride;
        const int Ho = (H - 1) / s + 1, Wo = (W - 1) / s + 1;
        if (s == 1 && !b.has_down && C == 32 && b.c1.oc == 32) {
            // the whole block in one launch; its intermediate stays in LDS
            if (profiling_) {
                const double npix = (double)batch * H * W;
                prof_begin("conv_block3x3_32", 2.0 * 2.0 * 9 * C * C * npix,
                           2.0 * (2.0 * npix * C + 2.0 * 9 * C * C) + 8.0 * C);
            }
            check(vdk_resblock3x3(x, batch, H, W, C, b.c1.w, b.c1.b, b.c2.w, b.c2.b, y, stream_));
            prof_end();
            xi = others[2];
            continue;
        }
        conv(b.c1, x, batch, H, W, nullptr, 1, h);
        const void* sc = x;
        if (b.has_down) {
            conv(b.down, x, batch, H, W, nullptr, 0, d);
            sc = d;
        }
        conv(b.c2, h, batch, Ho, Wo, sc, 1, y);
        xi = others[2];
        C = b.c1.oc;
        H = Ho;
        W = Wo;
    }
    prof_begin("tstp", 0.0, 2.0 * batch * (double)H * W * C + 4.0 * batch * pooled_dim_);
    check(vdk_tstp(ws_.act[xi], batch, H, W, C, cfg_.resnet.var_eps, ws_.pooled, stream_));
    prof_end();
    embed_fc("linear", ws_.pooled, batch, pooled_dim_, seg_w_, seg_b_, mean_vec_, cfg_.embedding_dim);
}

void Model::embed_batch_device(const float* d_pcm, int batch, int n_samples, float* d_out) {
    std::lock_guard<std::mutex> lock(mu_);
    require(batch > 0, "voicedetect: batch must be positive");
    require(d_pcm && d_out, "voicedetect: NULL device pointer");
    require(!is_analyzer(), "voicedetect: this model has no speaker embedding head (an analyze model)");
    check_frames(n_samples);
    ensure_device();
    ensure_workspace(batch, n_samples);
    forward(d_pcm, batch, n_samples, d_out);
}

void Model::embed_capture(const float* pcm, int batch, int n_samples, float* feats, float* pooled,
                          float* pre_norm, float* out) {
    std::lock_guard<std::mutex> lock(mu_);
    require(batch > 0 && pcm, "voicedetect: invalid pcm batch");
    require(!is_analyzer(), "voicedetect: this model has no speaker embedding head (an analyze model)");
    check_frames(n_samples);
    ensure_device();
    ensure_workspace(batch, n_samples);
    const size_t E = (size_t)cfg_.embedding_dim;
    if (!copy_pool_) {
        const unsigned hw = std::thread::hardware_concurrency();
        copy_pool_.reset(new CopyPool((int)std::min(3u, hw > 1 ? hw / 2 : 0u)));
    }
    stage_h2d(*copy_pool_, pin_in_, ws_.pcm, pcm, batch, sizeof(float) * (size_t)n_samples, 8, stream_);
    forward(ws_.pcm, batch, n_samples, ws_.emb);
    const size_t T = (size_t)frames(n_samples);
    if (feats) {   // the features as vdk_fbank gives them: with the CMN subtraction
        if (ws_.fb_mean) check(vdk_fbank_sub_mean(ws_.feats, ws_.fb_mean, batch, cfg_.fbank.n_mels, (int)T, stream_));
        VDK_HIP(hipMemcpyAsync(feats, ws_.feats, sizeof(float) * batch * cfg_.fbank.n_mels * T,
                               hipMemcpyDeviceToHost, stream_));
    }
    if (pooled)
        VDK_HIP(hipMemcpyAsync(pooled, ws_.pooled, sizeof(float) * batch * pooled_dim_, hipMemcpyDeviceToHost,
                               stream_));
    if (pre_norm)
        VDK_HIP(hipMemcpyAsync(pre_norm, ws_.pre, sizeof(float) * batch * E, hipMemcpyDeviceToHost, stream_));
    float* const eo = out ? static_cast<float*>(pin_out_.get(sizeof(float) * batch * E)) : nullptr;
    if (out) VDK_HIP(hipMemcpyAsync(eo, ws_.emb, sizeof(float) * batch * E, hipMemcpyDeviceToHost, stream_));
    VDK_HIP(hipStreamSynchronize(stream_));
    if (out) std::memcpy(out, eo, sizeof(float) * batch * E);
}

void Model::embed_batch_host(const float* pcm, int batch, int n_samples, float* out) {
    embed_capture(pcm, batch, n_samples, nullptr, nullptr, nullptr, out);
}

std::vector<float> Model::embed_pcm(const std::vector<float>& pcm, int sample_rate) {
    require(!is_analyzer(), "voicedetect: this model has no speaker embedding head (an analyze model)");
    const std::vector<float> x = sample_rate == 16000 ? pcm : resample_linear(pcm, sample_rate, 16000);
    check_frames((int)x.size());
    std::vector<float> out((size_t)cfg_.embedding_dim);
    embed_batch_host(x.data(), 1, (int)x.size(), out.data());
    return out;
}

void Model::synchronize() {
    std::lock_guard<std::mutex> lock(mu_);
    if (stream_) VDK_HIP(hipStreamSynchronize(stream_));
}

hipStream_t Model::stream() {
    std::lock_guard<std::mutex> lock(mu_);
    ensure_device();
    return stream_;
}

void Model::set_profiling(bool on, const std::string& name_prefix) {
    std::lock_guard<std::mutex> lock(mu_);
    profiling_ = on;
    prof_filter_ = name_prefix;
}

void Model::set_profiling_markers(bool on) {
    std::lock_guard<std::mutex> lock(mu_);
    ensure_device();
    if (on && !prof_marker_) VDK_HIP(hipMalloc(&prof_marker_, 256));
    prof_markers_ = on;
}

std::vector<ProfileRecord> Model::take_profile() {
    std::lock_guard<std::mutex> lock(mu_);
    std::vector<ProfileRecord> out;
    if (stream_) VDK_HIP(hipStreamSynchronize(stream_));
    for (auto& p : pending_) {
        float ms = 0.0f;
        VDK_HIP(hipEventElapsedTime(&ms, p.a, p.b));
        out.push_back({p.name, p.flops, p.bytes, (double)ms});
        event_pool_.push_back(p.a);
        event_pool_.push_back(p.b);
    }
    pending_.clear();
    return out;
}

}  // namespace vdk
