// model_campplus.cpp - the CAM++ encoder of vdk::Model (src/encoder_campplus.cpp:148-320).
//
// Device layout:
//   FCM      NHWC f16 [B][freq][T][m_ch]; the stem is the f32 single-channel
//            3x3 kernel, the residual blocks run on the implicit-GEMM conv with
//            a frequency-only stride (stride_h = 2, stride_w = 1); the final
//            freq-stride-2 conv stores time-major [B][T][freq][m_ch], i.e. the
//            [T][320] TDNN input with channel h*m_ch + c (the TDNN weight's input
//            channels are permuted from the reference's c*H + h at load).
//   backbone time-major f16 [B][T'][C]; each dense block keeps one buffer wide
//            enough for its final width, every layer appending its growth
//            channels in place (the reference's concat).  Per layer: linear1
//            1x1 (+ReLU) with the layer's BN+ReLU applied to its operand as it
//            is fetched (the normalised map is never stored) -> one launch per
//            (clip, 100-frame segment) for the CAM layer: segment sums,
//            context MLP (one gate per clip and segment) and the k=3 dilated
//            linear_local with the gate applied to its outputs.  The transit
//            convs fold their BN+ReLU the same way.
//   head     stats pooling (mean, unbiased std, no eps) -> dense 1x1 with the
//            affine-free BatchNorm folded in -> L2.
// Weights: conv weights f16 [OC][KH][KW][IC] (Q8_0 / F16 / F32 dequantised at
// load), the context MLP and the dense head f32.
#include <algorithm>
#include <utility>
#include <cmath>
#include <string>

#include "arena.hpp"
#include "common.hpp"
#include "model.hpp"
#include "weights.hpp"

namespace vdk {

namespace {

constexpr int kCamLayers[3] = {12, 24, 16};   // src/encoder_campplus.cpp:197-198
constexpr int kCamDil[3] = {1, 2, 2};
constexpr int kCamSeg = 100;                   // context segment length (src/encoder_campplus.cpp:170-182)

}  // namespace

void Model::upload_campplus() {
    const GgufFile& g = *gguf_;
    const CamPPlusCfg& cp = cfg_.campplus;
    Campplus& m = campp_;
    ArenaBuilder arena;
    require(cp.conv_weight.size() == cp.conv_bias.size(), "voicedetect: campplus conv manifests differ in length");
    const int n_conv_expect = 12 + 1 + 4 * (kCamLayers[0] + kCamLayers[1] + kCamLayers[2]) + 3 + 1;
    require((int)cp.conv_weight.size() == n_conv_expect && cp.bn_prefix.size() == 55,
            "voicedetect: campplus manifest does not match the 225-conv / 55-BN topology");
    int ci = 0, bi = 0;
    auto f32v = [&](const std::string& name, size_t n) {
        std::vector<float> v = g.to_f32(name);
        require(v.size() == n, "voicedetect: tensor '" + name + "' has the wrong size");
        return v;
    };
    auto bias = [&](int idx, int oc, float** dst) {
        if (cp.conv_bias[idx].empty()) { *dst = nullptr; return; }
        arena.put(f32v(cp.conv_bias[idx], oc), dst);
    };
    auto conv = [&](int ic_expect, int icp, Layer& l, const std::function<int(int)>& map = nullptr) {
        const int idx = ci++;
        const HostConv c = read_conv(g, cp.conv_weight[idx]);
        require(c.ic == ic_expect, "voicedetect: '" + cp.conv_weight[idx] + "' has " + std::to_string(c.ic) +
                                       " input channels, expected " + std::to_string(ic_expect));
        require(c.oc % 8 == 0, "voicedetect: '" + cp.conv_weight[idx] + "' needs a multiple of 8 output channels");
        l.ic = icp; l.oc = c.oc; l.kh = c.kh; l.k = c.kw;
        arena.put(pack_conv_f16(c, icp, map), &l.w);
        bias(idx, c.oc, &l.b);
        return c;
    };
    auto bn = [&](int C, float** s, float** t) {
        const std::string p = cp.bn_prefix[bi++];
        const std::vector<float> ga = f32v(p + ".weight", C), be = f32v(p + ".bias", C),
                                 mu = f32v(p + ".running_mean", C), var = f32v(p + ".running_var", C);
        std::vector<float> sc(C), sh(C);
        for (int i = 0; i < C; ++i) {   // src/encoder_campplus.cpp:125-130
            sc[i] = ga[i] / std::sqrt(var[i] + cp.bn_eps);
            sh[i] = be[i] - sc[i] * mu[i];
        }
        arena.put(sc, s);
        arena.put(sh, t);
    };

    // FCM stem: [m_ch, 1, 3, 3] f32 for the single-channel kernel
    {
        const HostConv c = read_conv(g, cp.conv_weight[0]);
        require(c.ic == 1 && c.kh == 3 && c.kw == 3, "voicedetect: campplus stem must be a 1-channel 3x3 conv");
        require(c.oc == 16 || c.oc == 32 || c.oc == 64, "voicedetect: campplus stem OC must be 16, 32 or 64");
        require(!cp.conv_bias[0].empty(), "voicedetect: campplus stem needs its folded bias");
        m.m_ch = c.oc;
        arena.put(c.w, &m.stem_w);
        bias(0, c.oc, &m.stem_b);
        ci = 1;
    }
    m.n_mels = cfg_.fbank.n_mels;
    m.fcm.assign(8 + 2, Layer());
    // (c1, c2, shortcut) for the stride-2 blocks, (c1, c2) for the stride-1 ones
    int li = 0;
    for (int stride : {2, 1, 2, 1}) {
        const int n = stride != 1 ? 3 : 2;
        for (int j = 0; j < n; ++j) {
            const HostConv& c = conv(m.m_ch, m.m_ch, m.fcm[li++]);
            require(c.oc == m.m_ch, "voicedetect: campplus FCM convs must keep the channel count");
        }
    }
    conv(m.m_ch, m.m_ch, m.fcm_out);
    int H = m.n_mels;
    for (int i = 0; i < 3; ++i) H = (H - 1) / 2 + 1;
    m.hf = H;
    const int fc = m.m_ch * m.hf;
    require(fc % 16 == 0, "voicedetect: campplus FCM output width must be a multiple of 16");
    // TDNN input channel c*hf + h of the reference lives at h*m_ch + c here
    const int mch = m.m_ch, hf = m.hf;
    require(!cp.conv_bias[ci].empty(), "voicedetect: campplus TDNN needs its folded bias");
    conv(fc, fc, m.tdnn, [mch, hf](int i) { return (i % hf) * mch + i / hf; });
    require(m.tdnn.k == 5 && m.tdnn.kh == 1, "voicedetect: campplus TDNN must be a k=5 conv1d");

    int C = m.tdnn.oc;
    for (int b = 0; b < 3; ++b) {
        CamBlock& blk = m.blocks[b];
        blk.dil = kCamDil[b];
        blk.layers.assign(kCamLayers[b], CamDense());
        for (int l = 0; l < kCamLayers[b]; ++l) {
            CamDense& d = blk.layers[l];
            d.c_in = C;
            require(C % 32 == 0, "voicedetect: campplus dense widths must be multiples of 32");
            bn(C, &d.bn_s, &d.bn_t);
            conv(C, C, d.l1);
            m.bn_ch = d.l1.oc;
            const HostConv& lc = conv(m.bn_ch, m.bn_ch, d.local);
            require(lc.kw == 3 && lc.kh == 1, "voicedetect: campplus linear_local must be a k=3 conv1d");
            m.growth = lc.oc;
            require(m.growth == 32 && m.bn_ch % 16 == 0 && m.bn_ch <= 256,
                    "voicedetect: campplus needs growth 32 and a bottleneck of 16..256 channels (multiple of 16)");
            // context MLP in f32 (dequantised)
            const int i1 = ci++, i2 = ci++;
            const HostConv c1 = read_conv(g, cp.conv_weight[i1]);
            const HostConv c2 = read_conv(g, cp.conv_weight[i2]);
            require(c1.ic == m.bn_ch && c1.kh * c1.kw == 1 && c2.ic == c1.oc && c2.oc == m.growth &&
                        c2.kh * c2.kw == 1, "voicedetect: campplus CAM linears have unexpected shapes");
            d.h1 = c1.oc;
            arena.put(c1.w, &d.c1_w);
            bias(i1, c1.oc, &d.c1_b);
            arena.put(c2.w, &d.c2_w);
            bias(i2, c2.oc, &d.c2_b);
            C += m.growth;
        }
        blk.cmax = C;
        bn(C, &blk.bn_s, &blk.bn_t);
        conv(C, C, blk.transit);
        C = blk.transit.oc;
    }
    m.c_out = C;
    // dense head + affine-free BN: y = (W x + b - mu) / sqrt(var + eps)
    {
        const int idx = ci++;
        const HostConv c = read_conv(g, cp.conv_weight[idx]);
        require(c.ic == 2 * C && c.kh * c.kw == 1 && c.oc == cfg_.embedding_dim,
                "voicedetect: campplus dense head must be 1x1 from 2*C to embedding_dim");
        const int E = c.oc, P = 2 * C;
        const std::vector<float> mu = f32v(cp.emb_bn_mean, E), var = f32v(cp.emb_bn_var, E);
        std::vector<float> b0(E, 0.0f);
        if (!cp.conv_bias[idx].empty()) b0 = f32v(cp.conv_bias[idx], E);
        std::vector<float> wf((size_t)E * P), bf(E);
        for (int o = 0; o < E; ++o) {
            const float inv = 1.0f / std::sqrt(var[o] + cp.bn_eps);
            for (int i = 0; i < P; ++i) wf[(size_t)o * P + i] = c.w[(size_t)o * P + i] * inv;
            bf[o] = b0[o] * inv + (0.0f - inv * mu[o]);
        }
        arena.put(wf, &m.dense_w);
        arena.put(bf, &m.dense_b);
    }
    require(ci == (int)cp.conv_weight.size() && bi == (int)cp.bn_prefix.size(),
            "voicedetect: campplus manifest walk did not consume every conv / BN");
    pooled_dim_ = 2 * m.c_out;
    arena_ = arena.upload();
}

void Model::alloc_campplus_workspace(int batch, int T) {
    const Campplus& m = campp_;
    Workspace& w = ws_;
    const int Tp = (T - 1) / 2 + 1;
    const size_t BTp = (size_t)batch * Tp;
    for (int i = 0; i < 3; ++i) w.fcm[i] = ws_alloc(2 * (size_t)batch * m.n_mels * T * m.m_ch);
    w.fcm_t = ws_alloc(2 * (size_t)batch * T * m.hf * m.m_ch);
    int cmax = 0;
    for (int b = 0; b < 3; ++b) {
        w.dense[b] = ws_alloc(2 * BTp * m.blocks[b].cmax);
        cmax = std::max(cmax, m.blocks[b].cmax);
    }
    w.cc = ws_alloc(2 * BTp * m.bn_ch);
    w.cc2 = ws_alloc(2 * BTp * m.bn_ch);
    w.segsum_bytes = 8 * (size_t)batch * ((Tp + kCamSeg - 1) / kCamSeg) * m.bn_ch;
    w.segsum[0] = static_cast<double*>(ws_alloc(w.segsum_bytes));
    w.segsum[1] = static_cast<double*>(ws_alloc(w.segsum_bytes));
    w.fin = ws_alloc(2 * BTp * m.c_out);
    w.fc_work_bytes = vdk_linear_workspace_size(batch, pooled_dim_, cfg_.embedding_dim);
    w.fc_work = ws_alloc(w.fc_work_bytes);
}

void Model::conv_ex(const char* name, const vdk_conv_desc& d) {
    if (profiling_) {
        const int sh = d.stride_h ? d.stride_h : 1, sw = d.stride_w ? d.stride_w : 1;
        const int dh = d.dil_h ? d.dil_h : 1, dw = d.dil_w ? d.dil_w : 1;
        const int Ho = (d.H + 2 * d.pad_h - (d.KH - 1) * dh - 1) / sh + 1;
        const int Wo = d.out_w > 0 ? d.out_w : (d.W + 2 * d.pad_w - (d.KW - 1) * dw - 1) / sw + 1;
        const double npix = (double)d.batch * Ho * Wo;
        const double flops = 2.0 * d.KH * d.KW * d.IC * (double)d.OC * npix;
        const double halves = d.split ? 2.0 : 1.0;   // split-f16 moves hi and lo
        const double bytes = 2.0 * halves * ((double)d.batch * d.H * d.W * d.IC + npix * d.OC * (d.residual ? 2.0 : 1.0)) +
                             2.0 * (d.split ? 3.0 : 1.0) * (double)d.OC * d.KH * d.KW * d.IC;
        prof_begin((std::string("conv.") + name).c_str(), flops, bytes);
    }
    check_rc(vdk_conv2d_ex(&d, stream_));
    prof_end();
}

void Model::encode_campplus(int batch, int T) {
    const Campplus& m = campp_;
    Workspace& w = ws_;
    const int Tp = (T - 1) / 2 + 1;
    const int nseg = (Tp + kCamSeg - 1) / kCamSeg;
    const long rows = (long)batch * Tp;

    // FCM (src/encoder_campplus.cpp:200-231)
    int H = m.n_mels;
    prof_begin("campp_stem3x3", 2.0 * 9 * m.m_ch * (double)batch * H * T,
               4.0 * batch * H * T + 2.0 * batch * H * T * m.m_ch);
    check_rc(vdk_stem_conv3x3_ex(w.feats, w.fb_mean, batch, H, T, m.stem_w, m.stem_b, m.m_ch, 1, 0, w.fcm[0],
                                 stream_));
    prof_end();
    auto fconv = [&](const char* name, const Layer& l, const void* x, int Hin, int sh, int pad, const void* res,
                     int relu, void* y) {
        vdk_conv_desc d{};
        d.x = x; d.batch = batch; d.H = Hin; d.W = T; d.IC = l.ic;
        d.w = l.w; d.OC = l.oc; d.KH = l.kh; d.KW = l.k;
        d.stride_h = sh; d.stride_w = 1; d.pad_h = d.pad_w = pad;
        d.bias = l.b; d.residual = res; d.act = relu ? VDK_ACT_RELU : VDK_ACT_NONE;
        d.y = y; d.tile = -1;
        conv_ex(name, d);
    };
    int cur = 0, li = 0;
    for (int stride : {2, 1, 2, 1}) {
        const int o1 = (cur + 1) % 3, o2 = (cur + 2) % 3;
        const int Ho = (H - 1) / stride + 1;
        const Layer& c1 = m.fcm[li++];
        const Layer& c2 = m.fcm[li++];
        if (stride != 1) {
            fconv("campp_fcm_conv1", c1, w.fcm[cur], H, stride, 1, nullptr, 1, w.fcm[o1]);
            const Layer& sc = m.fcm[li++];
            fconv("campp_fcm_shortcut", sc, w.fcm[cur], H, stride, 0, nullptr, 0, w.fcm[o2]);
            fconv("campp_fcm_conv2", c2, w.fcm[o1], Ho, 1, 1, w.fcm[o2], 1, w.fcm[cur]);
        } else if (c1.ic == 32 && c1.oc == 32 && c2.oc == 32 && c1.kh == 3 && c1.k == 3 && c2.kh == 3 && c2.k == 3) {
            // the identity block as one fused launch (conv1 -> ReLU -> conv2 -> + x -> ReLU,
            // the intermediate kept on chip; the same bits as the two convs)
            prof_begin("campp_fcm_block", 2.0 * 2 * 9 * 32 * 32 * (double)batch * H * T,
                       2.0 * 2 * 32 * (double)batch * H * T);
            check_rc(vdk_resblock3x3(w.fcm[cur], batch, H, T, 32, c1.w, c1.b, c2.w, c2.b, w.fcm[o2], stream_));
            prof_end();
            cur = o2;
        } else {
            fconv("campp_fcm_conv1", c1, w.fcm[cur], H, stride, 1, nullptr, 1, w.fcm[o1]);
            fconv("campp_fcm_conv2", c2, w.fcm[o1], Ho, 1, 1, w.fcm[cur], 1, w.fcm[o2]);
            cur = o2;
        }
        H = Ho;
    }
    {
        vdk_conv_desc d{};
        d.x = w.fcm[cur]; d.batch = batch; d.H = H; d.W = T; d.IC = m.fcm_out.ic;
        d.w = m.fcm_out.w; d.OC = m.fcm_out.oc; d.KH = 3; d.KW = 3;
        d.stride_h = 2; d.stride_w = 1; d.pad_h = d.pad_w = 1;
        d.bias = m.fcm_out.b; d.act = VDK_ACT_RELU;
        d.y = w.fcm_t; d.y_time_major = 1; d.tile = -1;
        conv_ex("campp_fcm_out", d);
    }

    // TDNN k=5 s2 p2 -> ReLU into the first dense buffer (src/encoder_campplus.cpp:236-239)
    auto tconv = [&](const char* name, const Layer& l, const void* x, int xs, int W, int sw, int pad, int dil,
                     const float* gate, int act, void* y, int ys, const float* in_scale = nullptr,
                     const float* in_shift = nullptr, double* seg_sum = nullptr) {
        vdk_conv_desc d{};
        d.in_scale = in_scale; d.in_shift = in_shift;
        d.seg_sum = seg_sum; d.seg_len = seg_sum ? kCamSeg : 0;
        d.x = x; d.batch = batch; d.H = 1; d.W = W; d.IC = l.ic; d.x_stride = xs;
        d.w = l.w; d.OC = l.oc; d.KH = 1; d.KW = l.k;
        d.stride_h = 1; d.stride_w = sw; d.pad_w = pad; d.dil_w = dil;
        d.bias = l.b; d.act = act;
        if (gate) { d.gate = gate; d.gate_seg = kCamSeg; d.gate_nseg = nseg; }
        d.y = y; d.y_stride = ys; d.tile = -1;
        conv_ex(name, d);
    };
    tconv("campp_tdnn", m.tdnn, w.fcm_t, m.tdnn.ic, T, 2, 2, 1, nullptr, VDK_ACT_RELU, w.dense[0], m.blocks[0].cmax);

    // dense blocks (src/encoder_campplus.cpp:250-281).  A block's first
    // linear1 runs as a conv that adds its output's per-(clip, segment) sums
    // to a cleared buffer (the CAM context's pooling, exact in f64); then
    // each launch runs one layer's CAM and the next layer's linear1 over the
    // same (clip, segment) (vdk_cam_dense: the next layer's input at a frame
    // is the block buffer plus the 32 channels just written), writing that
    // linear1's output h into the other h buffer and its segment sums into
    // the other sums buffer; the block's last CAM runs alone and clears the
    // buffer the next block's first linear1 accumulates into.
    VDK_HIP(hipMemsetAsync(w.segsum[0], 0, w.segsum_bytes, stream_));
    VDK_HIP(hipMemsetAsync(w.segsum[1], 0, w.segsum_bytes, stream_));
    int p = 0;   // the sums buffer of the current h
    for (int b = 0; b < 3; ++b) {
        const CamBlock& blk = m.blocks[b];
        uint8_t* D = static_cast<uint8_t*>(w.dense[b]);
        void* h = w.cc;
        void* hn = w.cc2;
        const int L = (int)blk.layers.size();
        for (int l = 0; l < L; ++l) {
            const CamDense& d = blk.layers[l];
            double* seg = w.segsum[p];
            double* seg_next = w.segsum[p ^ 1];
            if (l == 0) {
                // nonlinear1 BN + ReLU (src/encoder_campplus.cpp:110-134) folded into
                // linear1's operand loads
                tconv("campp_linear1", d.l1, D, blk.cmax, Tp, 1, 0, 1, nullptr, VDK_ACT_RELU, h, m.bn_ch, d.bn_s,
                      d.bn_t, seg);
            }
            const CamDense* dn = l + 1 < L ? &blk.layers[l + 1] : nullptr;
            // (measured at 32 x 10 s: the launch pair 19.4 / 22.1 / 25.9 / 27.9 / 32.3 us against 17.0 / 20.6 /
            // 24.5 / 29.2 / 34.7 us in one for 160 / 352 / 544 / 768 / 1024 input channels: the linear1 conv
            // streams wide inputs faster on its 500 workgroups, so only narrow layers take the one launch)
            const bool fuse = dn && m.bn_ch == 128 && m.growth == 32 && d.c_in % 32 == 0 && dn->c_in == d.c_in + 32 &&
                              dn->c_in <= 544 && dn->l1.k == 1 && dn->l1.oc == 128 && dn->l1.b && dn->bn_s;
            if (fuse) {
                prof_begin("campp_cam_dense",
                           2.0 * rows * 3 * m.bn_ch * m.growth +
                               2.0 * batch * nseg * ((double)d.h1 * m.bn_ch + (double)m.growth * d.h1) +
                               2.0 * rows * dn->c_in * m.bn_ch,
                           2.0 * rows * m.bn_ch * (1.0 + nseg) + 2.0 * rows * m.growth +
                               2.0 * rows * (dn->c_in + m.bn_ch));
                check_rc(vdk_cam_dense(h, batch, Tp, kCamSeg, blk.dil, d.c1_w, d.c1_b, d.h1, d.c2_w, d.c2_b,
                                       d.local.w, d.local.b, D, blk.cmax, d.c_in, seg, dn->l1.w, dn->l1.b, dn->bn_s,
                                       dn->bn_t, hn, seg_next, stream_));
                prof_end();
                std::swap(h, hn);
                p ^= 1;
                continue;
            }
            // the CAM layer alone: context from the segment sums, mask MLP and the gated
            // linear_local in one launch; it clears the other sums buffer
            prof_begin("campp_cam_local",
                       2.0 * rows * 3 * m.bn_ch * m.growth +
                           2.0 * batch * nseg * ((double)d.h1 * m.bn_ch + (double)m.growth * d.h1),
                       2.0 * rows * m.bn_ch * (1.0 + nseg) + 2.0 * rows * m.growth);
            check_rc(vdk_cam_local(h, m.bn_ch, batch, Tp, m.bn_ch, kCamSeg, blk.dil, d.c1_w, d.c1_b, d.h1, d.c2_w,
                                   d.c2_b, d.local.w, d.local.b, D + 2 * (size_t)d.c_in, blk.cmax, seg, seg_next,
                                   stream_));
            prof_end();
            p ^= 1;
            if (dn) {   // the next layer's linear1 as a conv into the cleared buffer
                tconv("campp_linear1", dn->l1, D, blk.cmax, Tp, 1, 0, 1, nullptr, VDK_ACT_RELU, h, m.bn_ch,
                      dn->bn_s, dn->bn_t, w.segsum[p]);
            }
        }
        const bool last = b == 2;
        tconv("campp_transit", blk.transit, D, blk.cmax, Tp, 1, 0, 1, nullptr, last ? VDK_ACT_RELU : VDK_ACT_NONE,
              last ? w.fin : w.dense[b + 1], last ? m.c_out : m.blocks[b + 1].cmax, blk.bn_s, blk.bn_t);
    }

    // stats pooling: mean + unbiased std, no eps (src/encoder_campplus.cpp:284-296)
    prof_begin("campp_stats", 0.0, 2.0 * rows * m.c_out + 8.0 * batch * m.c_out);
    check_rc(vdk_tstp(w.fin, batch, 1, Tp, m.c_out, 0.0f, w.pooled, stream_));
    prof_end();
    embed_fc("campp_dense", w.pooled, batch, pooled_dim_, m.dense_w, m.dense_b, nullptr, cfg_.embedding_dim);
}

}  // namespace vdk
