// model.hpp - load-once speaker-embedding context on one MI355X.
//
// Counterpart of vd::Model (src/model.hpp:18-57): parses the GGUF once on the
// host (no GPU needed), and on the first embed uploads the weights into one
// device arena in kernel-ready layouts and creates the context's HIP stream.
// Every embed runs the whole path on the GPU (FBank -> encoder -> pooling ->
// FC -> L2) for a batch of equal-length clips.  A context is driven by one
// caller at a time; an internal mutex serialises concurrent calls.
#pragma once

#include <hip/hip_runtime.h>

#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "gguf.hpp"
#include "hoststage.hpp"
#include "vdk.h"

namespace vdk {

// head.hip: the marker dispatch of Model::set_profiling_markers.
void launch_profile_marker(int* p, int v, hipStream_t s);

struct ResNetCfg {
    std::string stem_weight, stem_bias;
    std::vector<std::string> conv1_weight, conv1_bias, conv2_weight, conv2_bias, down_weight, down_bias;
    std::vector<int32_t> stride;
    std::string seg_weight, seg_bias, mean_vec;
    float var_eps = 1e-8f;
};

// src/model_loader.hpp:82-99
struct CamPPlusCfg {
    std::vector<std::string> conv_weight, conv_bias, bn_prefix;
    std::string emb_bn_mean, emb_bn_var;
    float bn_eps = 1e-5f;
};

// src/model_loader.hpp:68-79
struct ERes2NetCfg {
    std::vector<std::string> conv_weight, conv_bias;
    std::vector<int32_t> conv_stride, num_blocks;
    int m_channels = 0, scale = 2;
    std::string seg_weight, seg_bias;
    float relu_clamp = 20.0f, var_eps = 1e-8f;
};

// wav2vec2 analyze models, `voicedetect.w2v2.*` (src/model_loader.hpp:112-135).
struct W2v2Cfg {
    int hidden = 0, n_layers = 0, n_heads = 0, ff = 0;
    std::vector<int32_t> conv_dims, conv_kernels, conv_strides;
    std::string feat_extract_norm, feat_extract_activation, hidden_act;
    bool conv_bias = false, do_normalize = false, stable_layer_norm = false, weighted_layer_sum = false;
    float eps = 1e-5f;
    int pos_k = 0, pos_groups = 0, pos_norm_dim = 2, proj = 0;
};

struct ModelConfig {
    std::string arch;
    int embedding_dim = 0;
    bool l2_normalize = true;
    bool analyze_present = false;
    vdk_fbank_cfg fbank{};
    ResNetCfg resnet;
    CamPPlusCfg campplus;
    ERes2NetCfg eres2net;
    W2v2Cfg w2v2;
    std::vector<std::string> emotion_labels, gender_labels;   // src/model_loader.hpp:140-142
};

// Throws vdk::Error with vdk_last_error() when a vdk_* call returned nonzero.
void check_rc(int rc);

struct ProfileRecord {
    std::string name;
    double flops = 0.0, bytes = 0.0, ms = 0.0;
};

class Model {
public:
    // Throws vdk::Error on a missing/malformed GGUF or a missing required key.
    static std::unique_ptr<Model> load(const std::string& path);
    ~Model();

    const ModelConfig& config() const { return cfg_; }
    int embedding_dim() const { return cfg_.embedding_dim; }
    // 2 * C * H' of the pooled statistics (known once the weights are on the device).
    int pooled_dim() const { return pooled_dim_; }

    // 16 kHz (resampled if needed) mono PCM -> L2-normalised embedding.
    std::vector<float> embed_pcm(const std::vector<float>& pcm, int sample_rate);
    // batch x n_samples host PCM (16 kHz) -> batch x dim host embeddings.
    void embed_batch_host(const float* pcm, int batch, int n_samples, float* out);
    // Device-resident batch on this context's stream; returns without waiting.
    void embed_batch_device(const float* d_pcm, int batch, int n_samples, float* d_out);
    // Same as embed_batch_host, also copying intermediate results (NULL = skip):
    // feats [B][n_mels][T], pooled [B][P], pre_norm [B][dim].
    void embed_capture(const float* pcm, int batch, int n_samples, float* feats, float* pooled,
                       float* pre_norm, float* out);
    void synchronize();
    hipStream_t stream();

    // ---- wav2vec2 analyze models (arch wav2vec2_emotion / wav2vec2_age_gender) ----
    bool is_analyzer() const;
    // Raw head outputs per clip: emotion logits, or [age_raw, gender logits...].
    int analyze_outputs() const;
    // Frames T' after the conv feature encoder for n samples (0 if too short).
    int analyze_frames(int n_samples) const;
    int analyze_hidden() const { return cfg_.w2v2.hidden; }
    int analyze_feat_dim() const { return cfg_.w2v2.conv_dims.empty() ? 0 : cfg_.w2v2.conv_dims.back(); }
    // batch x n_samples host PCM (16 kHz) -> batch x analyze_outputs() host raw outputs.
    void analyze_batch_host(const float* pcm, int batch, int n_samples, float* raw);
    // Device-resident batch on this context's stream; returns without waiting.
    void analyze_batch_device(const float* d_pcm, int batch, int n_samples, float* d_raw);
    // Same as analyze_batch_host, also copying (NULL = skip) the conv features
    // [B][T'][feat_dim] and the last hidden state [B][T'][hidden].
    void analyze_capture(const float* pcm, int batch, int n_samples, float* feat, float* hidden, float* raw);
    // The reference's analyze JSON for one clip (src/analyze_w2v2.cpp:561-594, 632-668).
    std::string analyze_json(const std::vector<float>& pcm, int sample_rate);

    void set_profiling(bool on, const std::string& name_prefix = std::string());
    // While profiling: bracket every recorded launch with a one-thread marker
    // dispatch (profile_marker_kernel), so a counter-collection run can tell
    // which dispatches belong to which record.
    void set_profiling_markers(bool on);
    // Waits for the stream and returns the per-launch records since the last call.
    std::vector<ProfileRecord> take_profile();

    Model(const Model&) = delete;
    Model& operator=(const Model&) = delete;

private:
    Model() = default;
    struct Conv {
        int ic = 0, oc = 0, k = 0, stride = 1, pad = 0;
        void* w = nullptr;     // f16 [OC][K][K][IC]
        void* wc = nullptr;    // chunk-major copy [IC/16][K*K][OC][16] (stride-1 3x3, OC % 128 == 0)
        float* b = nullptr;    // f32 [OC]
    };
    struct Block {
        Conv c1, c2, down;
        bool has_down = false;
    };
    // A conv1d / 1x1 layer of the TDNN encoders on the implicit-GEMM kernels
    // (time is the W axis, H = 1): y = bn(relu(conv(x) + b)) with the eval
    // BatchNorm as a per-channel affine after the activation.
    struct Layer {
        int ic = 0, oc = 0, k = 1, kh = 1;
        int split = 1;              // split-f16 weight terms: 1 = [hi|hi|lo], 2 = [hi|hi] (exact in f16)
        void* w = nullptr;          // f16 [OC][KH][K][IC]
        void* wc = nullptr;         // chunk-major copy of w (split-f16 3x3 layers; may be null)
        float* b = nullptr;         // f32 [OC]
        float* scale = nullptr;     // BatchNorm after ReLU (nullptr = none)
        float* shift = nullptr;
    };
    struct EcapaBlock {
        Layer tdnn1, tdnn2;
        std::vector<Layer> res;     // scale - 1 dilated k=3 group convs
        float* se1_w = nullptr;     // f32 [se][C]
        float* se1_b = nullptr;
        float* se2_w = nullptr;     // f32 [C][se]
        float* se2_b = nullptr;
        int se_ch = 0, dil = 1;
    };
    struct Ecapa {
        int n_mels = 0, c_pad0 = 0, C = 0, scale = 0, group = 0, mfa = 0, att = 0;
        Layer block0, mfa_l, asp_x, asp_conv;
        std::vector<EcapaBlock> blocks;
        float* asp_stats_w = nullptr;   // f32 [att][2*mfa]: the global-context columns of asp.tdnn
        float* asp_b = nullptr;
        float* fc_w = nullptr;          // fc with asp_bn folded in, f32 [E][2*mfa]
        float* fc_b = nullptr;
    };
    // CAM++ (src/encoder_campplus.cpp): FCM convs, strided TDNN, three dense
    // blocks of context-masked layers with halving transits, stats, dense head.
    struct CamDense {
        float* bn_s = nullptr;      // nonlinear1 BN as scale / shift over c_in
        float* bn_t = nullptr;
        Layer l1, local;            // 1x1 c_in -> bn_ch (+ReLU); k=3 bn_ch -> growth (gated)
        float* c1_w = nullptr;      // CAM context MLP, f32 [h1][bn_ch], [growth][h1]
        float* c1_b = nullptr;
        float* c2_w = nullptr;
        float* c2_b = nullptr;
        int c_in = 0, h1 = 0;
    };
    struct CamBlock {
        std::vector<CamDense> layers;
        float* bn_s = nullptr;      // transit nonlinear BN
        float* bn_t = nullptr;
        Layer transit;
        int dil = 1, cmax = 0;
    };
    struct Campplus {
        int n_mels = 0, m_ch = 0, hf = 0, bn_ch = 0, growth = 0, c_out = 0;
        float* stem_w = nullptr;    // f32 [m_ch][9]
        float* stem_b = nullptr;
        std::vector<Layer> fcm;     // FCM convs after the stem, manifest order
        Layer fcm_out;              // final 3x3 freq-stride-2 conv
        Layer tdnn;                 // k=5 s2 over [B][T][hf*m_ch] (channels in (h, c) order)
        CamBlock blocks[3];
        float* dense_w = nullptr;   // head with the affine-free BN folded, f32 [E][2*c_out]
        float* dense_b = nullptr;
    };
    // ERes2Net (src/encoder_eres2net.cpp).  A block's conv1 output and its two
    // chunk outputs share one [.. 4w] buffer laid out [chunk0 | chunk1 | sp0 | sp1]
    // so that every concatenation the block needs is a contiguous channel slice.
    struct EresAff { Layer c1, c2; };   // local_att: 1x1 -> SiLU -> 1x1 -> tanh
    struct EresBlock {
        Layer conv1;      // 1x1, block stride, -> 2w, clamp
        Layer conv_a;     // chunk 0: 3x3 over [chunk0 (| chunk1 with zero weights when w % 32 != 0)]
        Layer conv_b;     // chunk 1: 3x3 over [chunk1 | sp0] with weights [W | W] (sum folded into the GEMM),
                          // or over the AFF output (diff_AFF blocks)
        bool aff = false;
        EresAff fuse;     // AFF(sp0, chunk1); conv1 input order [chunk1 | sp0]
        Layer conv3;      // 1x1 over [sp0 | sp1] -> 2*planes (+ residual, clamp)
        // 16-channel chunks with f16-exact conv_a / conv_b weights: both convs
        // run as one launch (vdk_res2_pair3x3) from these f16 [16][3][3][16] copies
        void* pair_a = nullptr;
        void* pair_b = nullptr;
        bool has_sc = false;
        Layer sc;         // 1x1 shortcut, block stride
        int stride = 1, width = 0, planes = 0, in_c = 0;
    };
    struct Eres2net {
        int m = 0, n_mels = 0, c_out = 0, h_out = 0;
        float clamp = 20.0f, eps = 1e-8f;
        float* stem_w = nullptr;   // f32 [m][9]
        float* stem_b = nullptr;
        std::vector<EresBlock> layers[4];
        Layer down[3];             // cross-stage 3x3 stride-2 downsamples (no bias)
        EresAff cross[3];          // cross-stage AFF(layer output, downsample)
        float* seg_w = nullptr;    // f32 [E][2*c_out*h_out]
        float* seg_b = nullptr;
    };
    // wav2vec2: every f16 matrix in the implicit-GEMM layout [OC][K][IC].
    struct W2Norm { float* g = nullptr; float* b = nullptr; };
    struct W2Layer {
        Layer qkv, out, ff1, ff2;   // qkv: q, k, v weights stacked [3H][H]
        W2Norm ln1, ln2;            // layer_norm, final_layer_norm
    };
    struct W2v2 {
        float* conv0_w = nullptr;   // f32 [C0][K0]
        float* conv0_b = nullptr;
        W2Norm conv0_n;
        std::vector<Layer> convs;   // conv layers 1.. (k = kernel, stride in strides)
        std::vector<W2Norm> conv_n; // their LayerNorms ("layer" feature norm)
        W2Norm fp_n;                // feature_projection.layer_norm
        Layer proj;
        // weight norm applied; vdk_pos_conv: one f16 [G][64][K][icg] array;
        // otherwise per group f16 [icg][K][icp] (input channels zero padded)
        std::vector<void*> pos_w;
        int pos_icp = 0;
        bool pos_fused = false;
        float* pos_b = nullptr;
        W2Norm enc_n;
        std::vector<W2Layer> layers;
        std::vector<float> state_w; // softmax(layer_weights) per hidden state (host)
        float *head_w1 = nullptr, *head_b1 = nullptr, *head_w2 = nullptr, *head_b2 = nullptr;   // projector / classifier
        float *age_w1 = nullptr, *age_b1 = nullptr, *age_w2 = nullptr, *age_b2 = nullptr;
        float *gen_w1 = nullptr, *gen_b1 = nullptr, *gen_w2 = nullptr, *gen_b2 = nullptr;
        int n_out = 0;
    };
    struct Workspace {
        int batch = 0, n_samples = 0;
        std::vector<void*> allocs;      // every allocation below, freed together
        size_t act_bytes = 0;
        float* pcm = nullptr;
        float* feats = nullptr;         // log-mel energies before CMN (the consumers subtract fb_mean)
        float* fb_mean = nullptr;       // [B][n_mels] CMN means, or NULL without CMN
        void* fb_work = nullptr;        // vdk_fbank_ex workspace (per-workgroup CMN sums)
        size_t fb_work_bytes = 0;
        void* act[4] = {nullptr, nullptr, nullptr, nullptr};
        float* pooled = nullptr;
        float* pre = nullptr;
        float* emb = nullptr;
        void* fc_work = nullptr;
        size_t fc_work_bytes = 0;
        // ECAPA: time-major f16 activations and f32 per-clip vectors
        void *x0p = nullptr, *h0 = nullptr, *t1 = nullptr, *t2 = nullptr, *s2b[2] = {nullptr, nullptr}, *cat = nullptr,
             *mfa = nullptr, *a1 = nullptr;
        float *logits = nullptr, *se_m = nullptr, *se_h = nullptr, *se_g = nullptr, *stats = nullptr,
              *pb = nullptr;
        // CAM++
        void* fcm[3] = {nullptr, nullptr, nullptr};
        void* fcm_t = nullptr;
        void* dense[3] = {nullptr, nullptr, nullptr};
        void *cc = nullptr, *cc2 = nullptr, *fin = nullptr;   // CAM++: linear1 outputs (two layers' worth)
        double* segsum[2] = {nullptr, nullptr};   // per-(clip, segment) sums of linear1's output, two layers' worth
        size_t segsum_bytes = 0;
        // ERes2Net
        void *ex[2] = {nullptr, nullptr}, *es4 = nullptr, *esc = nullptr, *ez = nullptr,
             *ef = nullptr;
        void *ecat[3] = {nullptr, nullptr, nullptr}, *efuse[3] = {nullptr, nullptr, nullptr};
        // wav2vec2
        float *wstats = nullptr, *fe32 = nullptr, *z = nullptr, *acc = nullptr, *wpool = nullptr, *wt1 = nullptr,
              *wt2 = nullptr, *raw = nullptr;
        void *fe[2] = {nullptr, nullptr}, *u = nullptr, *wproj = nullptr, *wh = nullptr, *wh1 = nullptr,
             *qkv = nullptr, *att = nullptr, *ffb = nullptr, *c0_work = nullptr;
        size_t c0_work_bytes = 0;
        int feat_buf = 0;           // which fe[] holds the conv features after a forward
    };

    void ensure_device();
    void upload_resnet();
    void upload_ecapa();
    void upload_campplus();
    void upload_eres2net();
    void upload_w2v2();
    void ensure_workspace(int batch, int n_samples);
    void alloc_w2v2_workspace(int batch, int n_samples);
    void analyze_forward(const float* d_pcm, int batch, int n_samples, float* d_raw);
    void alloc_resnet_workspace(int batch, int T);
    void alloc_ecapa_workspace(int batch, int T);
    void alloc_campplus_workspace(int batch, int T);
    void alloc_eres2net_workspace(int batch, int T);
    void* ws_alloc(size_t bytes);
    void free_workspace();
    // The whole forward for device PCM into device embeddings (pre-norm copy in ws_.pre).
    void forward(const float* d_pcm, int batch, int n_samples, float* d_out);
    // Encoder from ws_.feats to ws_.pooled (raw pooling statistics) and ws_.pre.
    void encode_resnet(int batch, int T);
    void encode_ecapa(int batch, int T);
    void encode_campplus(int batch, int T);
    void encode_eres2net(int batch, int T);
    // One vdk_conv2d_ex launch with profiling (flops from the descriptor's shape).
    void conv_ex(const char* name, const vdk_conv_desc& d);
    void conv(const Conv& c, const void* x, int batch, int H, int W, const void* res, int relu, void* y);
    // Time-major TDNN layer: x [B][W][x_stride] (W = T + 2*pad of a pre-padded
    // input) -> y [B][W - (k-1)*dil][y_stride].
    void tdnn(const char* name, const Layer& l, const void* x, int x_stride, int batch, int W, int dil,
              const float* bias, int bias_bs, int relu, int tanh_after, void* y, int y_stride, int y_f32);
    void res2_conv(const Layer& l, const void* x, int x_stride, int batch, int T, int dil, void* y, int y_stride,
                   const void* r2, int r2_stride, void* y2);
    void linear(const char* name, const float* x, int batch, int in_dim, const float* w, const float* b,
                const float* mv, int out_dim, int relu, float* y);
    // The embedding FC into ws_.pre; with L2 normalisation the same launch
    // pair also writes the normalised rows to l2_dst_.
    void embed_fc(const char* name, const float* x, int batch, int in_dim, const float* w, const float* b,
                  const float* mv, int out_dim);
    void prof_begin(const char* name, double flops, double bytes);
    void prof_end();
    int frames(int n_samples) const;
    int min_frames() const;                 // fewest FBank frames the encoder accepts
    void check_frames(int n_samples) const; // throws for clips the encoder cannot take

    std::unique_ptr<GgufFile> gguf_;
    ModelConfig cfg_;
    std::mutex mu_;

    float* l2_dst_ = nullptr;   // forward's output while an encoder runs (L2 in the FC's reduce)
    bool ready_ = false;
    int device_ = 0;
    hipStream_t stream_ = nullptr;
    // host-buffer entry points: pinned staging of the PCM and of the results
    std::unique_ptr<CopyPool> copy_pool_;
    PinnedBuffer pin_in_, pin_out_;
    void* arena_ = nullptr;
    void* fb_tables_ = nullptr;
    float* stem_w_ = nullptr;
    float* stem_b_ = nullptr;
    int stem_oc_ = 0;
    std::vector<Block> blocks_;
    Ecapa ecapa_;
    Campplus campp_;
    Eres2net eres_;
    W2v2 w2_;
    float* seg_w_ = nullptr;
    float* seg_b_ = nullptr;
    float* mean_vec_ = nullptr;
    int pooled_dim_ = 0;
    Workspace ws_;

    bool profiling_ = false;
    std::string prof_filter_;   // record only launches whose name starts with this (empty: all)
    bool prof_open_ = false;    // the last prof_begin recorded a start event
    bool prof_markers_ = false; // marker dispatches around recorded launches
    int* prof_marker_ = nullptr;
    struct Pending { std::string name; double flops, bytes; hipEvent_t a, b; };
    std::vector<Pending> pending_;
    std::vector<hipEvent_t> event_pool_;
};

}  // namespace vdk
