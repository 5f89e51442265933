// model_eres2net.cpp - the ERes2Net encoder of vdk::Model (src/encoder_eres2net.cpp:139-265).
//
// Precision: with random-init weights this network amplifies f16 rounding of
// activations or weights about a hundredfold (pooled statistics move by ~4%
// under either alone), so it runs in split-f16: every activation is stored as
// hi + lo f16 halves, weights as [hi | hi | lo], and each conv computes
// x_hi.w_hi + x_lo.w_hi + x_hi.w_lo on f16 MFMA with f32 accumulation
// (~2^-21 relative per value; 3x the MFMA work and 2x the activation bytes).
//
// Device layout: NHWC, every tensor [B][freq][T][hi(C) | lo(C)]; a channel
// slice of a tensor is (base + c, pixel stride 2C, lo offset C).  Every conv
// is one implicit-GEMM launch with bias, residual and the Hardtanh(0, 20)
// clamp in its epilogue.  Per Res2Net block (width w, scale 2) one tensor holds
//   [chunk0 | chunk1 | sp0 | sp1]      (4w channels)
// so that: conv1 writes [chunk0 | chunk1]; the chunk-0 3x3 conv reads chunk0
// (or [chunk0 | chunk1] with zero weights on chunk1 when w is not a multiple
// of 32) and writes sp0; the chunk-1 input sp0 + chunk1 is folded into the
// GEMM by reading [chunk1 | sp0] with the weights duplicated; in the diff_AFF
// blocks AFF(sp0, chunk1) reads [chunk1 | sp0] with its first conv's input
// channels swapped; conv3 reads [sp0 | sp1].  A layer's last block writes the
// first half of a 2C-channel tensor whose second half receives the
// cross-stage downsample, so the cross-stage AFF reads its concatenation in
// place.  Weights: split f16 [OC][KH][KW][3*IC] (Q8_0 / F32 dequantised at
// load), or [OC][KH][KW][2*IC] for a layer whose weights f16 holds exactly
// (the x_hi . w_lo term is zero and is skipped); seg_1 f32.
#include <algorithm>
#include <cmath>
#include <string>

#include "arena.hpp"
#include "common.hpp"
#include "model.hpp"
#include "weights.hpp"

namespace vdk {

namespace {

// A channel slice of a split-f16 tensor.
struct View {
    void* p;
    int stride, lo;   // elements between pixels / from hi to lo
    int gn, gs;       // channels per group, elements between groups (gs == gn: channels contiguous)
    View at(int ch) const {
        return {static_cast<uint8_t*>(p) + 2 * ((size_t)(ch / gn) * gs + ch % gn), stride, lo, gn, gs};
    }
};

// [hi C | lo C] per pixel
View split_tensor(void* p, int channels) { return {p, 2 * channels, channels, 16, 16}; }
// [hi g | lo g] per g-channel group: a Res2Net chunk of g = 16 channels is
// one 64-byte piece of the pixel row, of 32 one 128-byte line, so the convs
// over layer 1 / 2's chunks read and write whole blocks
View grouped_tensor(void* p, int channels, int g) { return {p, 2 * channels, g, g, 2 * g}; }

}  // namespace

void Model::upload_eres2net() {
    const GgufFile& g = *gguf_;
    const ERes2NetCfg& ec = cfg_.eres2net;
    Eres2net& m = eres_;
    ArenaBuilder arena;
    const size_t nconv = ec.conv_weight.size();
    require(nconv > 0 && ec.conv_bias.size() == nconv && ec.conv_stride.size() == nconv,
            "voicedetect: eres2net conv manifests differ in length");
    require(ec.num_blocks.size() == 4, "voicedetect: eres2net needs 4 layers");
    require(ec.scale == 2, "voicedetect: eres2net Res2Net scale must be 2");
    m.m = ec.m_channels;
    m.n_mels = cfg_.fbank.n_mels;
    m.clamp = ec.relu_clamp;
    m.eps = ec.var_eps;
    size_t ci = 0;
    auto next = [&](int ic_expect, int k_expect, int stride_expect) {
        require(ci < nconv, "voicedetect: eres2net manifest has too few convs");
        const size_t idx = ci++;
        HostConv c = read_conv(g, ec.conv_weight[idx]);
        require(c.ic == ic_expect && c.kh == k_expect && c.kw == k_expect,
                "voicedetect: '" + ec.conv_weight[idx] + "' has an unexpected shape");
        require(ec.conv_stride[idx] == stride_expect,
                "voicedetect: '" + ec.conv_weight[idx] + "' has an unexpected stride");
        return std::make_pair(c, idx);
    };
    // split weights; oc_pad > oc adds zero output rows (and zero bias)
    auto put = [&](const HostConv& c, size_t idx, int icp, Layer& l, const std::function<int(int)>& map = nullptr,
                   int oc_pad = 0) {
        require(c.oc % 8 == 0, "voicedetect: eres2net conv widths must be multiples of 8");
        const int ocp = std::max(c.oc, oc_pad);
        l.ic = icp; l.oc = ocp; l.kh = c.kh; l.k = c.kw;
        // weights that f16 holds exactly need no x_hi . w_lo term
        const bool exact = conv_f16_exact(c);
        l.split = exact ? 2 : 1;
        const std::vector<uint16_t> packed = pack_conv_f16_split(c, icp, ocp, map, exact ? 2 : 3);
        arena.put(packed, &l.w);
        // the register-weight kernels load their A fragments from a
        // chunk-major copy as whole cache lines
        const int icw = (exact ? 2 : 3) * icp;
        if (c.kh == 3 && c.kw == 3 && icw % 16 == 0) {
            std::vector<uint16_t> chunked(packed.size());
            vdk_conv_pack_chunked(packed.data(), ocp, 3, 3, icw, chunked.data());
            arena.put(chunked, &l.wc);
        }
        if (!ec.conv_bias[idx].empty()) {
            std::vector<float> b = g.to_f32(ec.conv_bias[idx]);
            require(b.size() == (size_t)c.oc, "voicedetect: '" + ec.conv_bias[idx] + "' has the wrong size");
            b.resize(ocp, 0.0f);
            arena.put(b, &l.b);
        } else {
            l.b = nullptr;
        }
    };
    // AFF local_att over cat(x, ds); swap = the tensor holds [ds | x].  The
    // bottleneck is padded to a multiple of 32 channels (zero rows / columns)
    // so that both convs run on the split-f16 DMA kernel.
    auto aff = [&](int C, bool swap, EresAff& a) {
        auto p1 = next(2 * C, 1, 1);
        const int zc = (p1.first.oc + 31) / 32 * 32;
        put(p1.first, p1.second, 2 * C, a.c1,
            swap ? std::function<int(int)>([C](int i) { return i < C ? i + C : i - C; }) : nullptr, zc);
        auto p2 = next(p1.first.oc, 1, 1);
        require(p2.first.oc == C, "voicedetect: eres2net AFF must return its channel count");
        put(p2.first, p2.second, zc, a.c2);
    };

    {   // stem: 1 -> m, 3x3, f32 for the single-channel kernel
        auto st = next(1, 3, 1);
        require(st.first.oc == m.m, "voicedetect: eres2net stem width differs from m_channels");
        require(m.m == 16 || m.m == 32 || m.m == 64, "voicedetect: eres2net m_channels must be 16, 32 or 64");
        require(!ec.conv_bias[st.second].empty(), "voicedetect: eres2net stem needs its folded bias");
        arena.put(st.first.w, &m.stem_w);
        arena.put(g.to_f32(ec.conv_bias[st.second]), &m.stem_b);
    }
    int in_planes = m.m, H = m.n_mels;
    for (int li = 0; li < 4; ++li) {
        const int planes = m.m << li;
        const int stride = li == 0 ? 1 : 2;
        m.layers[li].assign(ec.num_blocks[li], EresBlock());
        for (int bi = 0; bi < ec.num_blocks[li]; ++bi) {
            EresBlock& b = m.layers[li][bi];
            b.stride = bi == 0 ? stride : 1;
            b.planes = planes;
            b.in_c = in_planes;
            b.aff = li >= 2;
            auto c1 = next(in_planes, 1, b.stride);
            put(c1.first, c1.second, in_planes, b.conv1);
            const int w = c1.first.oc / 2;
            b.width = w;
            require(w % 8 == 0, "voicedetect: eres2net chunk width must be a multiple of 8");
            // chunk 0: [chunk0 (| chunk1 zero-weighted)]; 16 channels alone when
            // the weights are f16-exact (the split-f16 register-weight kernel)
            auto ca = next(w, 3, 1);
            put(ca.first, ca.second, (w % 32 == 0 || (w == 16 && conv_f16_exact(ca.first))) ? w : 2 * w, b.conv_a);
            if (b.aff) {
                aff(w, true, b.fuse);
                auto cb = next(w, 3, 1);
                put(cb.first, cb.second, w, b.conv_b);
            } else {
                // [chunk1 | sp0] with the weights on both halves: conv(sp0 + chunk1)
                auto cb = next(w, 3, 1);
                if (w == 16 && conv_f16_exact(ca.first) && conv_f16_exact(cb.first)) {
                    arena.put(pack_conv_f16(ca.first, w), &b.pair_a);
                    arena.put(pack_conv_f16(cb.first, w), &b.pair_b);
                }
                HostConv dup = cb.first;
                dup.ic = 2 * w;
                dup.w.assign((size_t)dup.oc * 2 * w * 9, 0.0f);
                for (int o = 0; o < dup.oc; ++o)
                    for (int half = 0; half < 2; ++half)
                        std::copy(cb.first.w.begin() + (size_t)o * w * 9, cb.first.w.begin() + (size_t)(o + 1) * w * 9,
                                  dup.w.begin() + ((size_t)o * 2 * w + (size_t)half * w) * 9);
                put(dup, cb.second, 2 * w, b.conv_b);
            }
            auto c3 = next(2 * w, 1, 1);
            require(c3.first.oc == 2 * planes, "voicedetect: eres2net conv3 must produce 2*planes channels");
            put(c3.first, c3.second, 2 * w, b.conv3);
            b.has_sc = b.stride != 1 || in_planes != 2 * planes;
            if (b.has_sc) {
                auto sc = next(in_planes, 1, b.stride);
                require(sc.first.oc == 2 * planes, "voicedetect: eres2net shortcut width differs");
                put(sc.first, sc.second, in_planes, b.sc);
            }
            in_planes = 2 * planes;
        }
        if (li > 0) H = (H - 1) / 2 + 1;
        if (li >= 1) {
            // cross-stage: downsample of the previous fused feature (3x3 s2, no bias), then AFF
            auto dn = next(planes, 3, 2);
            require(dn.first.oc == 2 * planes && ec.conv_bias[dn.second].empty(),
                    "voicedetect: eres2net cross-stage downsample must be a bias-free 3x3 to 2*planes");
            put(dn.first, dn.second, planes, m.down[li - 1]);
            aff(2 * planes, false, m.cross[li - 1]);
        }
    }
    require(ci == nconv, "voicedetect: eres2net manifest has unused convs");
    m.c_out = in_planes;
    m.h_out = H;
    pooled_dim_ = 2 * m.c_out * m.h_out;
    {
        std::vector<float> sw = g.to_f32(ec.seg_weight);
        require(sw.size() == (size_t)cfg_.embedding_dim * pooled_dim_,
                "voicedetect: eres2net seg_1 must be [embedding_dim, 2*C*H']");
        arena.put(sw, &m.seg_w);
        std::vector<float> sb = g.to_f32(ec.seg_bias);
        require(sb.size() == (size_t)cfg_.embedding_dim, "voicedetect: eres2net seg_1 bias has the wrong size");
        arena.put(sb, &m.seg_b);
    }
    arena_ = arena.upload();
}

void Model::alloc_eres2net_workspace(int batch, int T) {
    const Eres2net& m = eres_;
    Workspace& w = ws_;
    size_t x_max = 0, s4_max = 0, z_max = 0, f_max = 0;   // channels x pixels (one half)
    int H = m.n_mels, W = T;
    for (int li = 0; li < 4; ++li) {
        if (li > 0) { H = (H - 1) / 2 + 1; W = (W - 1) / 2 + 1; }
        const size_t pix = (size_t)batch * H * W;
        x_max = std::max(x_max, pix * m.m);   // stem output
        for (const EresBlock& b : m.layers[li]) {
            x_max = std::max(x_max, pix * 2 * b.planes);
            s4_max = std::max(s4_max, pix * 4 * b.width);
            if (b.aff) {
                z_max = std::max(z_max, pix * std::max(b.fuse.c1.oc, b.fuse.c2.oc));
                f_max = std::max(f_max, pix * b.width);
            }
        }
        if (li >= 1) {
            const int C = 2 * (m.m << li);
            w.ecat[li - 1] = ws_alloc(2 * 2 * pix * 2 * C);
            w.efuse[li - 1] = ws_alloc(2 * 2 * pix * C);
            z_max = std::max(z_max, pix * std::max(m.cross[li - 1].c1.oc, m.cross[li - 1].c2.oc));
        }
    }
    // split-f16: two f16 halves per value
    w.ex[0] = ws_alloc(4 * x_max);
    w.ex[1] = ws_alloc(4 * x_max);
    w.esc = ws_alloc(4 * x_max);
    w.es4 = ws_alloc(4 * s4_max);
    w.ez = ws_alloc(4 * std::max<size_t>(z_max, 8));
    w.ef = ws_alloc(4 * std::max<size_t>(f_max, 8));
    w.fc_work_bytes = vdk_linear_workspace_size(batch, pooled_dim_, cfg_.embedding_dim);
    w.fc_work = ws_alloc(w.fc_work_bytes);
}

void Model::encode_eres2net(int batch, int T) {
    const Eres2net& m = eres_;
    Workspace& w = ws_;
    const View* aff_x = nullptr;    // AFF combine operands of the next conv (the second local_att conv)
    const View* aff_ds = nullptr;
    auto conv = [&](const char* name, const Layer& l, View x, int H, int W, int stride, const View* res, int act,
                    float clamp, int tanh_after, View y) {
        vdk_conv_desc d{};
        d.x = x.p; d.batch = batch; d.H = H; d.W = W; d.IC = l.ic; d.x_stride = x.stride;
        d.w = l.w; d.w_chunked = l.wc; d.OC = l.oc; d.KH = l.kh; d.KW = l.k;
        d.stride_h = d.stride_w = stride;
        d.pad_h = (l.kh - 1) / 2; d.pad_w = (l.k - 1) / 2;
        d.bias = l.b;
        if (res) {
            require(res->gs == res->gn, "voicedetect: eres2net residuals are contiguous split tensors");
            d.residual = res->p; d.res_stride = res->stride; d.res_lo = res->lo;
        }
        d.act = act; d.clamp_hi = clamp; d.tanh_after = tanh_after;
        d.y = y.p; d.y_stride = y.stride;
        d.split = l.split; d.x_lo = x.lo; d.y_lo = y.lo;
        d.x_group = x.gn; d.x_group_stride = x.gs; d.y_group = y.gn; d.y_group_stride = y.gs;
        if (aff_x) {
            d.aff_x = aff_x->p; d.aff_x_stride = aff_x->stride; d.aff_x_lo = aff_x->lo;
            d.aff_ds = aff_ds->p; d.aff_ds_stride = aff_ds->stride; d.aff_ds_lo = aff_ds->lo;
        }
        d.tile = -1;
        conv_ex(name, d);
    };
    // AFF(x, ds): local_att over the [.. 2C] input `cat`; the second conv's
    // epilogue applies tanh and the combine (x + ds) + t * (x - ds) into y
    auto aff = [&](const char* name, const EresAff& a, View cat, View x, View ds, int C, int H, int W, View y) {
        const View z = split_tensor(w.ez, a.c1.oc);
        conv(name, a.c1, cat, H, W, 1, nullptr, VDK_ACT_SILU, 0.0f, 0, z);
        require(x.gs == x.gn && ds.gs == ds.gn, "voicedetect: eres2net AFF operands are contiguous split tensors");
        aff_x = &x;
        aff_ds = &ds;
        conv(name, a.c2, z, H, W, 1, nullptr, VDK_ACT_NONE, 0.0f, 1, y);
        aff_x = aff_ds = nullptr;
    };

    int H = m.n_mels, W = T;
    prof_begin("eres_stem3x3", 2.0 * 9 * m.m * (double)batch * H * W, 4.0 * batch * H * W + 4.0 * batch * H * W * m.m);
    check_rc(vdk_stem_conv3x3_ex(w.feats, w.fb_mean, batch, H, W, m.stem_w, m.stem_b, m.m, 1, 1, w.ex[0], stream_));
    prof_end();
    View x = split_tensor(w.ex[0], m.m);
    int xi = 0;
    const float hi = m.clamp;
    // The cross-stage convs run as soon as their input exists (the manifest
    // order is only the load order): down[li] right after the map it reads.
    for (int li = 0; li < 4; ++li) {
        const int nb = (int)m.layers[li].size();
        for (int bi = 0; bi < nb; ++bi) {
            const EresBlock& b = m.layers[li][bi];
            const int Ho = (H - 1) / b.stride + 1, Wo = (W - 1) / b.stride + 1;
            const int wd = b.width;
            const View s4 = (wd == 16 || wd == 32) && !b.aff ? grouped_tensor(w.es4, 4 * wd, wd)
                                                             : split_tensor(w.es4, 4 * wd);
            const bool last = bi == nb - 1 && li >= 1;
            const View y = last ? split_tensor(w.ecat[li - 1], 4 * b.planes) : split_tensor(w.ex[xi ^ 1], 2 * b.planes);
            const bool pair = b.pair_a && s4.gn == 16;
            const bool pair_c3 = pair && b.conv3.kh * b.conv3.k == 1 && b.conv3.ic == 32 && b.conv3.oc == 64 &&
                                 y.gs == y.gn;
            // the whole block in one launch: stride 1, x contiguous
            // (the residual is x or the shortcut's split_tensor output: contiguous either way)
            const bool whole = pair_c3 && b.conv1.kh * b.conv1.k == 1 && b.conv1.split != 0 && b.stride == 1 &&
                               b.conv1.oc == 32 && (b.conv1.ic == 32 || b.conv1.ic == 64) && x.gs == x.gn &&
                               x.lo == b.conv1.ic && (b.has_sc || b.conv1.ic == 64);
            // conv1 -> [chunk0 | chunk1]
            if (!whole) conv("eres_conv1", b.conv1, x, H, W, b.stride, nullptr, VDK_ACT_RELU, hi, 0, s4);
            // the shortcut (its input is the block input: independent of the chunks)
            View res = x;
            if (b.has_sc) {
                res = split_tensor(w.esc, 2 * b.planes);
                conv("eres_shortcut", b.sc, x, H, W, b.stride, nullptr, VDK_ACT_NONE, 0.0f, 0, res);
            }
            if (whole) {
                // conv1, the pair and conv3 + residual in one launch; [c0 | c1] and sp0 / sp1 stay on chip
                const int terms = b.conv3.split == 2 ? 2 : 3;
                const int ic = b.conv1.ic;
                prof_begin("eres_res2_whole",
                           2.0 * ((double)32 * (b.conv1.split == 2 ? 2 : 3) * ic + 9 * 16 * 16 * 2 * 3 +
                                  64.0 * 32 * terms) * batch * Ho * Wo,
                           2.0 * (2 * ic + 2 * 64 + (b.has_sc ? 2 * 64 : 0)) * (double)batch * Ho * Wo);
                check_rc(vdk_res2_bottleneck(x.p, x.stride, x.lo, ic, batch, Ho, Wo, b.conv1.w,
                                             b.conv1.split == 2 ? 2 : 3, b.conv1.b, b.pair_a,
                                             b.conv_a.b, b.pair_b, b.conv_b.b, b.conv3.w, b.conv3.b, terms,
                                             b.has_sc ? res.p : nullptr, res.stride, res.lo, y.p, y.stride, y.lo, hi,
                                             stream_));
                prof_end();
            } else if (pair_c3 && res.gs == res.gn) {
                // chunk 0 -> sp0, chunk 1 (+ sp0) -> sp1 and conv3 + residual -> clamp in one launch
                // (MFMA work: conv_a 16 x 16 x 9 over both planes, conv_b twice that, conv3 64 x 32 per term)
                const int terms = b.conv3.split == 2 ? 2 : 3;
                prof_begin("eres_res2_block",
                           2.0 * ((double)9 * 16 * 16 * 2 * 3 + 64.0 * 32 * terms) * batch * Ho * Wo,
                           2.0 * (2 * 32 + 2 * 64 + 2 * 64) * (double)batch * Ho * Wo);
                check_rc(vdk_res2_pair3x3_conv3(s4.p, s4.stride, batch, Ho, Wo, b.pair_a, b.conv_a.b, b.pair_b,
                                                b.conv_b.b, b.conv3.w, b.conv3.b, terms, res.p, res.stride, res.lo,
                                                y.p, y.stride, y.lo, hi, stream_));
                prof_end();
            } else {
                if (pair) {
                    // chunk 0 -> sp0 and chunk 1 (+ sp0) -> sp1 in one launch
                    // MFMA work: conv_a 16 x 16 x 9 over both planes, conv_b the same twice (c1, sp0)
                    prof_begin("eres_res2_pair", 2.0 * 9 * 16 * 16 * 2 * 3 * (double)batch * Ho * Wo,
                               2.0 * 2 * 64 * (double)batch * Ho * Wo);
                    check_rc(vdk_res2_pair3x3(s4.p, s4.stride, s4.at(2 * wd).p, s4.stride, batch, Ho, Wo, b.pair_a,
                                              b.conv_a.b, b.pair_b, b.conv_b.b, hi, stream_));
                    prof_end();
                } else {
                    // chunk 0 -> sp0
                    conv("eres_conv3x3", b.conv_a, s4, Ho, Wo, 1, nullptr, VDK_ACT_RELU, hi, 0, s4.at(2 * wd));
                    // chunk 1 -> sp1
                    if (b.aff) {
                        const View f = split_tensor(w.ef, wd);
                        aff("eres_aff_block", b.fuse, s4.at(wd), s4.at(2 * wd), s4.at(wd), wd, Ho, Wo, f);
                        conv("eres_conv3x3", b.conv_b, f, Ho, Wo, 1, nullptr, VDK_ACT_RELU, hi, 0, s4.at(3 * wd));
                    } else {
                        conv("eres_conv3x3", b.conv_b, s4.at(wd), Ho, Wo, 1, nullptr, VDK_ACT_RELU, hi, 0,
                             s4.at(3 * wd));
                    }
                }
                // conv3 + residual -> clamp
                conv("eres_conv3", b.conv3, s4.at(2 * wd), Ho, Wo, 1, &res, VDK_ACT_RELU, hi, 0, y);
            }
            if (!last) xi ^= 1;
            x = y;
            H = Ho;
            W = Wo;
        }
        const int C = 2 * (m.m << li);   // this layer's output channels
        if (li >= 1) {
            // AFF(layer output, downsample) from the [out | down] tensor (src/encoder_eres2net.cpp:203-223)
            const View cat = split_tensor(w.ecat[li - 1], 2 * C);
            aff("eres_aff_cross", m.cross[li - 1], cat, cat, cat.at(C), C, H, W, split_tensor(w.efuse[li - 1], C));
        }
        if (li < 3) {
            // downsample of this stage's feature (layer 1 output, else the fused map) into the
            // second half of the next layer's [out | down] tensor
            const View src = li == 0 ? x : split_tensor(w.efuse[li - 1], C);
            conv("eres_downsample", m.down[li], src, H, W, 2, nullptr, VDK_ACT_NONE, 0.0f, 0,
                 split_tensor(w.ecat[li], 4 * C).at(2 * C));
        }
    }
    // TSTP over the last fused map, then seg_1 (src/encoder_eres2net.cpp:228-250)
    const View fin = split_tensor(w.efuse[2], m.c_out);
    prof_begin("eres_tstp", 0.0, 4.0 * batch * (double)H * W * m.c_out + 4.0 * batch * pooled_dim_);
    check_rc(vdk_tstp_ex(fin.p, fin.stride, fin.lo, batch, H, W, m.c_out, m.eps, w.pooled, stream_));
    prof_end();
    embed_fc("eres_seg1", w.pooled, batch, pooled_dim_, m.seg_w, m.seg_b, nullptr, cfg_.embedding_dim);
}

}  // namespace vdk
