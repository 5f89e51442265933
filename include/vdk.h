/*
 * vdk.h - low-level C ABI of the MI355X (gfx950) speaker-encoder kernels.
 *
 * Every entry point takes device pointers, plain sizes and a HIP stream
 * (`void* stream`, NULL = the default stream), enqueues its kernels and
 * returns 0, or a nonzero code with a message from vdk_last_error().  Nothing
 * here allocates device memory except vdk_malloc.  Shapes are checked on the
 * host before any launch.
 *
 * Layouts: PCM [B][n] f32; FBank features feat-major [B][n_mels][T] f32 (the
 * reference's [n_mels, T] per clip); activations NHWC f16 [B][H=freq][W=time][C];
 * conv weights [OC][KH][KW][IC] f16 (the reference's [OC][IC][KH][KW] with the
 * channel axis moved innermost); biases f32.
 *
 * These replace the reference's operator seam: the conv2d_auto router and the
 * ggml custom ops it dispatches to (src/backend.cpp:665-793), the host FBank
 * (src/fbank.cpp:121-205) and the ggml pooling / FC / host L2 tail of
 * src/encoder_resnet.cpp:140-183.
 */
#ifndef VDK_H
#define VDK_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- device memory helpers (for callers without another HIP runtime) ---- */
int         vdk_device_count(void);
int         vdk_set_device(int device);
void*       vdk_malloc(size_t bytes);          /* NULL on failure */
int         vdk_free(void* p);
int         vdk_memcpy_h2d(void* dst, const void* src, size_t bytes);
int         vdk_memcpy_d2h(void* dst, const void* src, size_t bytes);
int         vdk_memcpy_d2d(void* dst, const void* src, size_t bytes);
int         vdk_memset(void* dst, int value, size_t bytes);
int         vdk_synchronize(void);
const char* vdk_last_error(void);             /* thread-local; "" if none */

/* ---- host utilities (no GPU needed) ---- */
/* Decode a WAV, average channels, resample linearly to 16 kHz
 * (src/audio_io.cpp:25-38).  Returns the sample count (copies at most cap
 * samples into out; out may be NULL to query), or -1 on failure. */
long vdk_load_wav_16k(const char* path, float* out, long cap);
/* Linear resampler of src/audio_io.cpp:9-23; returns the output length
 * (copies at most cap samples). */
long vdk_resample_linear(const float* in, long n, int in_sr, int out_sr, float* out, long cap);
/* IEEE f32 -> f16 bit patterns, round to nearest even (weight packing). */
void vdk_f32_to_f16(const float* in, unsigned short* out, size_t n);

/* ---- FBank front end ----
 * Replaces vd::FBank::compute (src/fbank.cpp:121-205), batched: B clips of
 * n_samples each.  `tables` is a device block built by vdk_fbank_tables_size /
 * vdk_fbank_tables_fill (window, FFT twiddles, packed mel filters).  Output
 * feat-major [B][n_mels][T], T = 1 + (n_samples - win) / hop. */
typedef struct {
    int sample_rate, n_mels, n_fft, win_length, hop_length;
    float preemph, low_freq, high_freq; /* high_freq <= 0 means Nyquist */
    int cmn;
} vdk_fbank_cfg;

size_t vdk_fbank_tables_size(const vdk_fbank_cfg* cfg);
/* Computes the tables on the host and copies them to d_tables (synchronous). */
int    vdk_fbank_tables_fill(const vdk_fbank_cfg* cfg, void* d_tables);
int    vdk_fbank(const vdk_fbank_cfg* cfg, const void* d_tables, const float* d_pcm,
                 int batch, int n_samples, float* d_feats, void* stream);
/* Same with a caller workspace (CMN: vdk_fbank_workspace_size bytes,
 * 256-byte aligned; no initial contents needed).
 * d_mean == NULL: the features come out normalised, as vdk_fbank.
 * d_mean != NULL (and cfg->cmn): the features come out WITHOUT the CMN
 * subtraction and d_mean [B][n_mels] receives each clip's per-bin means, for
 * a consumer that subtracts them as it loads (vdk_stem_conv3x3_ex,
 * vdk_feats_tmajor: row mean arguments) or for vdk_fbank_sub_mean; the f32
 * values such a consumer sees are those vdk_fbank stores.  The means sum
 * the log-mel values of a clip as fixed-point 2^-36 integers, so the result
 * does not depend on how the frames are grouped into workgroups. */
size_t vdk_fbank_workspace_size(const vdk_fbank_cfg* cfg, int batch, int n_samples);
int    vdk_fbank_ex(const vdk_fbank_cfg* cfg, const void* d_tables, const float* d_pcm,
                    int batch, int n_samples, float* d_feats, float* d_mean,
                    void* d_work, size_t work_size, void* stream);
/* feats [B][n_mels][T] -= mean [B][n_mels] (the CMN subtraction, f32). */
int    vdk_fbank_sub_mean(float* d_feats, const float* d_mean, int batch, int n_mels, int T, void* stream);

/* ---- 2D convolution, implicit GEMM on f16 MFMA with f32 accumulation ----
 * Replaces the blocked-island ops blocked_conv3x3 / blocked_conv1x1 with their
 * fused bias(+ReLU) epilogue and blocked_add_relu (src/directconv.cpp:1496-1546,
 * src/directconv.hpp:22-51), and the per-conv directconv_conv3x3 / winograd
 * custom ops (src/directconv.cpp:1449-1458, src/winograd.cpp:638-648):
 *   y = act(conv(x, w) + bias [+ residual])
 * x [B][H][W][IC], w [OC][KH][KW][IC], bias [OC] (may be NULL),
 * residual [B][Ho][Wo][OC] (may be NULL), y [B][Ho][Wo][OC], all f16 except bias.
 * Ho = (H + 2*pad - KH)/stride + 1 (same for W).  Requires IC % 16 == 0 and
 * OC % 8 == 0.  relu: 0 = none, 1 = max(v, 0). */
int vdk_conv2d_nhwc(const void* d_x, int batch, int H, int W, int IC,
                    const void* d_w, int OC, int KH, int KW, int stride, int pad,
                    const float* d_bias, const void* d_residual, int relu,
                    void* d_y, void* stream);

/* Activations of the fused epilogues (conv and FC).  GELU is the exact erf
 * form x * Phi(x) (the wav2vec2 activation, src/analyze_w2v2.cpp:126-128). */
enum { VDK_ACT_NONE = 0, VDK_ACT_RELU = 1, VDK_ACT_SIGMOID = 2, VDK_ACT_SILU = 3, VDK_ACT_GELU = 4,
       VDK_ACT_TANH = 5 };

/* General form.  Pixel strides let a layer read or write a channel slice of a
 * wider NHWC tensor in place (pass the slice's base pointer; 0 means dense).
 * Stride, zero pad and dilation are per axis (0 stride / dilation means 1):
 * Ho = (H + 2*pad_h - (KH-1)*dil_h - 1)/stride_h + 1, likewise Wo.  A 1-D
 * time conv over a time-major [B][T][C] map is H = 1, W = T, KH = 1.
 * Epilogue, in order:
 *   v = acc + bias                 (bias_batch_stride > 0: clip b reads bias + b*stride)
 *   v *= gate[b][ow / gate_seg][oc]  (gate [B][gate_nseg][OC] f32, may be NULL)
 *   v += residual                  (f16, or f32 when res_f32)
 *   v = act(v)                     (RELU then min(v, clamp_hi) if clamp_hi > 0; SIGMOID; SILU; GELU)
 *   v += residual                  (instead of the add above when res_after_act)
 *   v = v*post_scale + post_shift  (a BatchNorm after the activation; may be NULL)
 *   v = tanh(v)                    (tanh_after)
 *   v = (x + ds) + v * (x - ds)    (aff_x / aff_ds: ERes2Net's AFF combine,
 *                                   src/encoder_eres2net.cpp:91-101; f16, or
 *                                   split-f16 with split, at the output pixel
 *                                   and channel, own pixel strides / lo offsets)
 * stored f16 (or f32 if y_f32) at pixel (b, oh, ow), or at (b, ow, oh) when
 * y_time_major (an NHWC [B][H][W][C] map written as [B][W][H*C], no residual).
 * in_scale / in_shift (1x1 convs without padding): the input channels pass
 * through relu(x * in_scale[c] + in_shift[c]), rounded to f16, on their way to
 * the MFMA (a standalone BatchNorm + ReLU before the conv, fused).
 * out_w > 0 keeps only the first out_w output columns of each row (a conv
 * whose right pad is one shorter than its left, e.g. wav2vec2's positional
 * conv with its last step dropped).  y and an f32 residual may be the same
 * buffer (each element is read before it is written, by the same thread).
 * OC needs only be a multiple of 8: surplus rows of a tile are masked.
 * w_chunked (may be NULL): the same weights re-ordered chunk-major,
 * [IC/16][KH*KW][OC][16] (vdk_conv_pack_chunked); kernels that stream 16-channel
 * weight chunks read it as whole cache lines.  Results do not depend on it.
 * split != 0 selects split-f16 arithmetic (~2^-21 relative instead of f16's
 * 2^-11, for ill-conditioned networks): x, residual and y hold value = hi + lo
 * with the lo halves x_lo / res_lo / y_lo elements after the hi halves (same
 * pixel strides).  split = 1: w is [OC][KH][KW][3*IC] = [hi | hi | lo] per tap
 * and the GEMM runs x_hi.w_hi + x_lo.w_hi + x_hi.w_lo on f16 MFMA (3x the
 * work); split = 2, for weights that f16 holds exactly (lo = 0): w is
 * [OC][KH][KW][2*IC] = [hi | hi] and the GEMM runs x_hi.w + x_lo.w (2x).
 * Split needs IC % 32 == 0, or IC = 16 with split = 2 (16 output channels,
 * 3x3 stride 1: the split-f16 register-weight kernel); a w_chunked copy of
 * split weights re-orders the [OC][KH][KW][terms*IC] array.
 * reflect_pad != 0 (1-D convs, KH = 1): the time axis is padded by reflection
 * without repeating the edge sample (x[-i] = x[i], x[W-1+i] = x[W-1-i],
 * SpeechBrain's padding, src/encoder.cpp:32-52) instead of with zeros; pad_w
 * must be below W.  y2 (may be NULL): a second f16 output y2 = v + res2 (v the
 * finished value above, res2 f16 at the same pixel, both with their own pixel
 * strides), e.g. the next Res2Net group's input y_j + x_{j+1}.
 * w_q8_0 (may be NULL; 1x1 convs with IC % 32 == 0, no split): the weights as
 * ggml q8_0 blocks straight from the model file, [OC][IC/32] blocks of 34
 * bytes (an f16 scale d, then 32 int8 quants q along IC), dequantised in the
 * kernel's registers to f16(q * d) (the product in f32: the f16 weights a
 * host dequantisation would store, so results equal those from w); w is then
 * not read.
 * seg_sum (may be NULL; H = 1 maps, f16 output, no split or time-major
 * store): the stored f16 outputs of each clip's segments of seg_len frames
 * (the last one may be shorter) are summed per channel and added to seg_sum
 * [B][ceil(W_out / seg_len)][OC] f64, which the caller zeroes; every term is
 * an f16, so the f64 sums are exact and independent of the order they are
 * added in (CAM++'s context pooling, src/encoder_campplus.cpp:159-170).
 * Register-staged tiles (f16 weights) whose pixel tile is at most seg_len wide.
 * x_group / y_group (16 or 32; 0: 16) and x_group_stride / y_group_stride
 * (0: the group size, channels contiguous): split-f16 tensors stored in
 * channel groups, channel c of the hi plane at element (c / group) *
 * group_stride + c % group of its pixel row (the lo plane x_lo / y_lo after
 * it); e.g. group 16, stride 32, lo 16 keeps each group's hi and lo halves as
 * one 64-byte piece ([hi 16 | lo 16]) and group 32, stride 64, lo 32 as one
 * 128-byte line, so channel slices are read and written as whole 64-byte
 * blocks or lines (narrower writes cost a read-modify-write in HBM, half-line
 * reads fetch whole lines).  IC / OC multiples of the group; the LDS-DMA and
 * split-f16 register-weight kernels.
 * tile = -1 picks the kernel automatically. */
typedef struct {
    const void* x; int batch, H, W, IC, x_stride;
    const void* w; int OC, KH, KW;
    int stride_h, stride_w, pad_h, pad_w, dil_h, dil_w;
    const float* bias; int bias_batch_stride;
    const float* gate; int gate_seg, gate_nseg;
    const void* residual; int res_stride;
    int act; float clamp_hi;
    const float* post_scale; const float* post_shift;
    int tanh_after;
    void* y; int y_stride, y_f32, y_time_major;
    int split; int x_lo, res_lo, y_lo;
    int tile;
    int res_f32, res_after_act, out_w;
    const float* in_scale; const float* in_shift;
    const void* w_chunked;
    int reflect_pad;
    void* y2; int y2_stride;
    const void* res2; int res2_stride;
    const void* w_q8_0;
    double* seg_sum; int seg_len;
    int x_group_stride, y_group_stride;
    int x_group, y_group;
    const void* aff_x; int aff_x_stride, aff_x_lo;
    const void* aff_ds; int aff_ds_stride, aff_ds_lo;
} vdk_conv_desc;
/* Host: tensor `name` of the GGUF file at `path` as f32 into out[n]
 * (n = the tensor's element count; F16 widened exactly, Q8_0 blocks
 * dequantised to q * d with the product in f32), the values every model
 * upload starts from (src/model_loader.cpp:114-215 reads the same file). */
int vdk_gguf_tensor_f32(const char* path, const char* name, float* out, long long n);
/* Host: re-order f16 conv weights [OC][KH][KW][IC] (IC % 16 == 0) into the
 * chunk-major [IC/16][KH*KW][OC][16] copy that vdk_conv_desc.w_chunked takes. */
void vdk_conv_pack_chunked(const unsigned short* w, int OC, int KH, int KW, int IC, unsigned short* out);
int vdk_conv2d_ex(const vdk_conv_desc* desc, void* stream);
/* Run-time tile tuning for vdk_conv2d_ex calls with tile = -1 (off by
 * default; VDK_CONV_AUTOTUNE=1 in the environment turns it on too).  No
 * reference counterpart: for conv shapes the built-in per-layer rules were
 * not measured on.  The first call of each shape (channels, kernel, strides,
 * map and batch size, epilogue features) times every tile that fits into
 * scratch outputs, keeps the fastest one whose output equals the default
 * tile's bit for bit, and synchronises the stream.  Later calls of the shape
 * use the cached choice.  Applies to plain f16 outputs that do not overlap
 * an input; others keep the default tile.  Not for use under stream capture
 * (the first call allocates).  Returns 0. */
int vdk_conv_set_autotune(int on);
/* The tile the tuner chose for this descriptor's shape, or -1 if it has not
 * tuned it. */
int vdk_conv_tuned_tile(const vdk_conv_desc* d);
int vdk_conv2d_tile_fits_ex(int tile, const vdk_conv_desc* desc);

/* Same contract with an explicit kernel/tile choice (index into the library's
 * tile table; vdk_conv2d_tile_fits tells which apply to a shape).  For
 * validation and tuning; vdk_conv2d_nhwc picks the tile itself. */
int vdk_conv2d_nhwc_tile(const void* d_x, int batch, int H, int W, int IC,
                         const void* d_w, int OC, int KH, int KW, int stride, int pad,
                         const float* d_bias, const void* d_residual, int relu,
                         void* d_y, void* stream, int tile);
int vdk_conv2d_tile_count(void);
int vdk_conv2d_tile_fits(int tile, int IC, int OC, int KH, int KW, int stride, int pad);

/* ---- fused stride-1 identity BasicBlock ----
 * Replaces one ResNet BasicBlock without downsample (src/encoder_resnet.cpp:33-48
 * basic_block / 50-73 basic_block_blocked: conv1 3x3 + bias -> ReLU -> conv2
 * 3x3 + bias -> + x -> ReLU, src/directconv.cpp:1364 blocked_add_relu) in one
 * launch whose intermediate map never leaves LDS:
 *   y = relu(conv2(relu(conv1(x) + b1)) + b2 + x)
 * x, y [B][H][W][C] f16 (must not overlap), w1, w2 [C][3][3][C] f16,
 * b1, b2 [C] f32; the intermediate is rounded to f16 as vdk_conv2d_nhwc stores
 * it.  C must be 32. */
int vdk_resblock3x3(const void* d_x, int batch, int H, int W, int C,
                    const void* d_w1, const float* d_b1, const void* d_w2, const float* d_b2,
                    void* d_y, void* stream);
/* Same with an explicit tile height (variant 0: 6 rows, 1: 4, 2: 8; -1 picks);
 * for validation and tuning. */
int vdk_resblock3x3_variant(const void* d_x, int batch, int H, int W, int C,
                            const void* d_w1, const float* d_b1, const void* d_w2, const float* d_b2,
                            void* d_y, int variant, void* stream);

/* ---- stem: single-input-channel 3x3 conv from f32 features ----
 * Replaces the ResNet stem conv2d_auto -> directconv_conv3x3 + bias + ReLU
 * (src/encoder_resnet.cpp:115-117).  feats [B][H][W] f32, w [OC][3][3] f32,
 * bias [OC] f32, y [B][H][W][OC] f16 (stride 1, pad 1), OC in {16, 32, 64}. */
int vdk_stem_conv3x3(const float* d_feats, int batch, int H, int W,
                     const float* d_w, const float* d_bias, int OC, int relu,
                     void* d_y, void* stream);
/* Same; split != 0 stores split-f16 [hi(OC) | lo(OC)] per pixel (see vdk_conv_desc);
 * d_row_mean (may be NULL): [B][H] subtracted from each in-map input value of
 * its row as it is loaded (the CMN means of vdk_fbank_ex). */
int vdk_stem_conv3x3_ex(const float* d_feats, const float* d_row_mean, int batch, int H, int W,
                        const float* d_w, const float* d_bias, int OC, int relu, int split,
                        void* d_y, void* stream);

/* ---- temporal statistics pooling ----
 * Replaces the TSTP graph of src/encoder_resnet.cpp:140-157: per (c, h) mean
 * over time and sqrt(unbiased var + eps), flattened C-outer/H-inner:
 * pooled[b] = [mean(c,h) ; std(c,h)], length 2*C*H.  x [B][H][W][C] f16. */
int vdk_tstp(const void* d_x, int batch, int H, int W, int C, float eps,
             float* d_pooled, void* stream);
/* Same over x with pixel stride x_stride (0 = C); x_lo > 0: split-f16 input,
 * value = x + x[.. + x_lo]. */
int vdk_tstp_ex(const void* d_x, int x_stride, int x_lo, int batch, int H, int W, int C, float eps,
                float* d_pooled, void* stream);

/* ---- embedding FC ----
 * Replaces the seg_1 mul_mat + bias - mean_vec of src/encoder_resnet.cpp:159-169:
 * y[b] = w x[b] + bias - mean_vec; w [out][in] f32; bias/mean_vec may be NULL.
 * d_work: caller-provided device workspace of at least
 * vdk_linear_workspace_size(batch, in_dim, out_dim) bytes (split-K partials;
 * the result is bitwise reproducible). */
size_t vdk_linear_workspace_size(int batch, int in_dim, int out_dim);
int vdk_linear(const float* d_x, int batch, int in_dim, const float* d_w,
               const float* d_bias, const float* d_mean_vec, int out_dim,
               float* d_y, void* d_work, size_t work_bytes, void* stream);
/* Same, with an activation on the result (act: VDK_ACT_NONE / RELU /
 * SIGMOID / TANH): the SE bottleneck of src/encoder.cpp:207-219, the ASP
 * global-context term, the CAM++ context MLP (src/encoder_campplus.cpp:266-267),
 * the age/gender ModelHead dense + tanh (src/analyze_w2v2.cpp:614-623). */
int vdk_linear_ex(const float* d_x, int batch, int in_dim, const float* d_w,
                  const float* d_bias, const float* d_mean_vec, int out_dim, int act,
                  float* d_y, void* d_work, size_t work_bytes, void* stream);
/* No counterpart in the reference.  vdk_linear_ex for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): the split-K partials live in a fixed
 * per-GPU array of VDK_LINEAR_SCRATCH_BYTES, held until the process ends, so
 * the call allocates nothing.  Fails (nothing launched) when
 * vdk_linear_workspace_size(batch, in_dim, out_dim) exceeds that size.  Every
 * call on one GPU shares its array: calls that overlap in time on one GPU
 * (e.g. on two streams) race; calls in one stream order do not.  Same result,
 * bit for bit, as vdk_linear_ex. */
#define VDK_LINEAR_SCRATCH_BYTES (4u << 20)
int vdk_linear_ex_noalloc(const float* d_x, int batch, int in_dim, const float* d_w,
                          const float* d_bias, const float* d_mean_vec, int out_dim, int act,
                          float* d_y, void* stream);

/* ---- ECAPA-TDNN helpers (src/encoder.cpp) ----
 * Activations are time-major f16 [B][T][stride] (channel slices by pointer
 * offset + stride; strides and channel counts of the half8 kernels are
 * multiples of 8 and pointers 16-byte aligned). */
/* FBank [B][n_mels][T] f32 -> [B][T+2*pad][c_pad] f16, reflect padded in time
 * without edge repeat (src/encoder.cpp:32-52) and zero channels n_mels..c_pad;
 * d_row_mean (may be NULL): [B][n_mels] CMN means subtracted as it loads. */
int vdk_feats_tmajor(const float* d_feats, const float* d_row_mean, int batch, int n_mels, int T, int pad,
                     int c_pad, void* d_out, void* stream);
/* All scale - 1 dependent group convs of one SE-Res2Net block's Res2Net
 * (src/encoder.cpp:174-200) in one launch.  buf [B][T][stride] f16 holds
 * the block's groups in slots of G channels: x_m (tdnn1's output chunk m) in
 * slot m + 1; group j (1 .. scale-1) = conv_j(in_j) with in_1 = x_1 and
 * in_j = f16(v_{j-1} + x_j), conv_j the k = 3 dilated conv with reflect
 * padding + bias -> ReLU -> BN (v = relu(conv + bias) * scale + shift, f32),
 * stored as f16 to slot 0 (j = 1) or slot j.  Weights [G][3][G] f16 (16-byte
 * aligned); scale / shift may be NULL (1 / 0).  The same bits as the groups
 * run one conv at a time (vdk_conv2d_ex with reflect_pad and the second
 * output).  G = 128, scale <= 8, T > dil, (scale - 1) * dil <= 64. */
typedef struct {
    const void* w[7]; const float* bias[7]; const float* scale[7]; const float* shift[7];
} vdk_res2_weights;
int vdk_res2_block(void* d_buf, int stride, int batch, int T, int G, int scale, int dil,
                   const vdk_res2_weights* w, void* stream);
/* out [B][T+2*pad][G] = reflect_pad(a (+ b)) over time: the Res2Net group
 * input x_i + y_{i-1} of src/encoder.cpp:174-200 padded for its dilated conv.
 * d_b may be NULL. */
int vdk_reflect_pad_add(const void* d_a, int a_stride, const void* d_b, int b_stride, int batch, int T,
                        int G, int pad, void* d_out, void* stream);
/* out [B][C] f32 = mean over time (SE squeeze, src/encoder.cpp:207-209), f64
 * sums; C, x_stride and d_x 8-channel (16-byte) aligned. */
int vdk_channel_mean(const void* d_x, int x_stride, int batch, int T, int C, float* d_out, void* stream);
/* y = x * sigmoid(gate[b][c]) + res (SE excitation and the block residual,
 * src/encoder.cpp:218-244). */
int vdk_se_gate_residual(const void* d_x, int x_stride, const float* d_gate, const void* d_res,
                         int res_stride, int batch, int T, int C, void* d_y, int y_stride, void* stream);
/* y = x * scale[b][c] + res: vdk_se_gate_residual with the sigmoid already
 * applied to the gate (once per clip and channel, e.g. by vdk_linear_ex's
 * VDK_ACT_SIGMOID, whose expression is the same, so y has the same bits). */
int vdk_se_scale_residual(const void* d_x, int x_stride, const float* d_scale, const void* d_res,
                          int res_stride, int batch, int T, int C, void* d_y, int y_stride, void* stream);
/* out [B][2C] = [mean_t x ; sqrt(max(var_t x, eps))] (ASP global context,
 * src/encoder.cpp:269-271): one pass of f64 sums of x and x^2, var =
 * E[x^2] - mean^2; C, x_stride and d_x 8-channel (16-byte) aligned. */
int vdk_asp_stats(const void* d_x, int x_stride, int batch, int T, int C, float eps, float* d_out,
                  void* stream);
/* softmax over time of logits [B][T][l_stride] f32 per channel, then
 * out [B][2C] = [sum a x ; sqrt(max(sum a (x-mu)^2, eps))] (src/encoder.cpp:282-294). */
int vdk_asp_pool(const float* d_logits, int l_stride, const void* d_x, int x_stride, int batch, int T,
                 int C, float eps, float* d_out, void* stream);
/* The asp.conv logits and the pooling of vdk_asp_pool in one launch
 * (src/encoder.cpp:283-294): l[b][t][c] = b_c[c] + sum_k w[c][k] a1[b][t][k]
 * (f16 products, f32 sums, the conv kernels' order), softmax over time per
 * channel, out [B][2C] = [sum a x ; sqrt(max(sum a (x-mu)^2, eps))]; the
 * logits never reach memory.  a1 [B][T][att] f16 dense (att = 128), w [C][att]
 * f16, b_c [C] f32, x [B][T][C] f16 dense, C % 64 == 0.  One pass over the
 * frames: the softmax normaliser and the weighted sums of x and x^2 are f64
 * with online rescaling of the running max; var = E_a[x^2] - mu^2 in f64. */
int vdk_asp_attn_pool(const void* d_a1, int a1_stride, const void* d_w, const float* d_b, int att,
                      const void* d_x, int x_stride, int batch, int T, int C, float eps, float* d_out,
                      void* stream);

/* ---- L2 normalisation ----
 * Replaces the host L2 of src/encoder_resnet.cpp:177-183 (double accumulation,
 * skipped when the norm is 0).  In place on x [B][dim]. */
/* The embedding FC with the L2 normalisation in its reduce step: d_pre
 * [B][out] the FC output as vdk_linear_ex (no activation) stores it, d_y the
 * rows of d_pre normalised as vdk_l2norm_to does (src/encoder_resnet.cpp:
 * 159-183); d_pre and d_y must not overlap. */
int vdk_linear_l2_ex(const float* d_x, int batch, int in_dim, const float* d_w, const float* d_bias,
                     const float* d_mean_vec, int out_dim, float* d_pre, float* d_y, void* d_work,
                     size_t work_bytes, void* stream);
int vdk_l2norm(float* d_x, int batch, int dim, void* stream);
/* Same, out of place: y [B][dim] = x / ||x|| (y may equal x; a zero row is copied). */
int vdk_l2norm_to(const float* d_x, int batch, int dim, float* d_y, void* stream);

/* ---- registry scoring: identify queries against enrolled embeddings ----
 * No counterpart in the reference's code: README.md:15 promises `identify`,
 * which no function or ABI symbol provides; the scoring follows its verify
 * (src/model.cpp:65-78, distance = 1 - sum(ea*eb) in double).
 * scores S[b][n] = sum_d q[b][d] * reg[n][d], each f32 x f32 product exact in
 * f64 and summed in f64; writes the k best rows per query (1 <= k <= 64,
 * k <= N) as idx[b][j] / score[b][j] (f32), highest first, equal scores by the
 * lower row index.  q [B][D], reg [N][D] f32 device (D % 4 == 0, 16-byte
 * aligned); d_work of at least vdk_registry_topk_workspace_size(B, N, k) bytes. */
size_t vdk_registry_topk_workspace_size(int B, int N, int k);
int vdk_registry_topk(const float* d_queries, int B, const float* d_registry, int N, int D, int k,
                      void* d_work, size_t work_bytes, int* d_idx, float* d_score, void* stream);

/* ---- CAM++ helpers (src/encoder_campplus.cpp) ---- */
/* y = act(x * scale[c] + shift[c]) over rows x C channels (the standalone
 * BatchNorm -> ReLU of each dense layer / transit, src/encoder_campplus.cpp:110-134). */
int vdk_bn_act(const void* d_x, int x_stride, long rows, int C, const float* d_scale,
               const float* d_shift, int act, void* d_y, int y_stride, void* stream);
/* out [B][nseg][C] f32: sums of x [B][T][x_stride] over each seg-frame segment
 * (nseg = ceil(T / seg)). */
int vdk_segment_sums(const void* d_x, int x_stride, int batch, int T, int C, int seg, float* d_out,
                     void* stream);
/* CAM context mask per (clip, segment) (src/encoder_campplus.cpp:159-182, 260-268):
 * ctx = sum_all / T + sum_seg / seg; gate = sigmoid(w2 relu(w1 ctx + b1) + b2),
 * w1 [H1][C], w2 [G][H1] f32; gate [B][nseg][G]. */
int vdk_cam_context(const float* d_sums, int batch, int T, int C, int seg, const float* d_w1,
                    const float* d_b1, int H1, const float* d_w2, const float* d_b2, int G,
                    float* d_gate, void* stream);
/* One dense layer's CAM layer in one launch (src/encoder_campplus.cpp:159-182,
 * 260-268): the context mask of vdk_cam_context computed per (clip, segment)
 * from x itself (its segment sums in f64), then
 * y = (linear_local(x) + bl) * gate, linear_local the k = 3 conv with
 * dilation dil and zero padding, C -> 32 channels, wl f16 [32][3][C]
 * (tap-major), bl [32] f32 (may be NULL); x [B][T][x_stride] f16 (C a
 * multiple of 16, 16..256), y [B][T][y_stride] f16 (the 32 outputs).
 * segsum (may be NULL): the f64 per-(clip, segment, channel) sums of x that
 * the conv producing x accumulated (vdk_conv_desc.seg_sum, seg_len = seg),
 * [B][ceil(T / seg)][C]; the context then comes from them instead of a pass
 * over x (same values: both sums are exact).  zero_next (may be NULL, needs
 * segsum): a buffer of the same shape that each (clip, segment) workgroup
 * clears, ready for the next layer's seg_sum. */
int vdk_cam_local(const void* d_x, int x_stride, int batch, int T, int C, int seg, int dil,
                  const float* d_w1, const float* d_b1, int H1, const float* d_w2, const float* d_b2,
                  const void* d_wl, const float* d_bl, void* d_y, int y_stride, const double* d_segsum,
                  double* d_zero_next, void* stream);

/* One dense layer's CAM (vdk_cam_local with C = 128 channels of h, its
 * context from segsum, zero_next NULL) and the next layer's linear1 in the
 * same launch, per (clip, segment) (src/encoder_campplus.cpp:250-281,
 * 110-134, 159-182): the CAM writes its 32 outputs into the block buffer
 * dense [B][T][dense_stride] at channel cin, then
 * hn = relu(wn . relu(dense[.., 0 : cin + 32] * scale_n + shift_n) + bn)
 * for the segment's frames (wn f16 [128][cin + 32], bn / scale_n / shift_n
 * f32; the prologue rounded to f16 as the GEMM operand) into hn [B][T][128],
 * and the segment's f64 sums of the stored hn values into its row of
 * seg_next [B][ceil(T / seg)][128] (stored, not added: nothing needs
 * clearing).  Equal bit for bit to vdk_cam_local followed by vdk_conv2d_ex's
 * linear1 with in_scale / in_shift and seg_sum.  h [B][T][128] f16 is read
 * with a dil-frame halo from the neighbouring segments, so hn must be
 * another buffer; cin % 32 == 0, cin + 32 <= 1024 and <= dense_stride,
 * seg <= 128.  A one-layer CAM++ block step in one launch instead of two. */
int vdk_cam_dense(const void* d_h, int batch, int T, int seg, int dil, const float* d_w1, const float* d_b1, int H1,
                  const float* d_w2, const float* d_b2, const void* d_wl, const float* d_bl, void* d_dense,
                  int dense_stride, int cin, const double* d_segsum, const void* d_wn, const float* d_bn,
                  const float* d_scale_n, const float* d_shift_n, void* d_hn, double* d_seg_next, void* stream);

/* ---- ERes2Net helper (src/encoder_eres2net.cpp:91-101) ----
 * AFF output y = (x + ds) + t * (x - ds) with t = tanh(local_att(cat(x, ds)))
 * already computed; all f16 rows of C channels with their own strides.  With
 * split != 0 every tensor is split-f16 (value = hi + lo, lo *_lo elements
 * after hi), as in vdk_conv_desc. */
int vdk_aff_combine(const void* d_t, int t_stride, int t_lo, const void* d_x, int x_stride, int x_lo,
                    const void* d_ds, int ds_stride, int ds_lo, long rows, int C, int split, void* d_y,
                    int y_stride, int y_lo, void* stream);

/* ERes2Net: the two chained Res2Net 3x3 convs of a plain (non-AFF) scale-2
 * block with 16-channel chunks (src/encoder_eres2net.cpp:111-137; layer 1 of
 * ERes2Net base), one launch, split-f16 with f16-exact weights:
 *   sp0 = min(relu(conv_a(c0) + b_a), clamp_hi),
 *   sp1 = min(relu(conv_b(sp0 + c1) + b_b), clamp_hi)   (clamp_hi <= 0: no clamp)
 * (3x3, stride 1, zero pad 1).  x: [batch][H][W] pixel rows of x_stride
 * elements whose first 64 hold c0, c1 as 16-channel groups [hi 16 | lo 16];
 * y: rows of y_stride elements whose first 64 receive sp0, sp1 the same way
 * (x and y may be slices of one buffer when they do not overlap).  w_a, w_b:
 * f16 [16][3][3][16]; b_a, b_b: f32 [16] (may be NULL).  Equal bit for bit to
 * vdk_conv2d_ex's split-f16 convs over the same slices (conv_b's input as the
 * 32 channels [c1 | sp0] with its weights on both halves).  16-byte aligned
 * pointers. */
int vdk_res2_pair3x3(const void* d_x, int x_stride, void* d_y, int y_stride, int batch, int H, int W,
                     const void* d_w_a, const float* d_b_a, const void* d_w_b, const float* d_b_b, float clamp_hi,
                     void* stream);

/* vdk_res2_pair3x3 followed by the block's conv3 in the same launch, sp0 and
 * sp1 never stored: y = min(relu(conv3([sp0 | sp1]) + b3 + res), clamp_hi),
 * 64 output channels, split-f16 (y and res: rows of *_stride elements, the
 * 64 hi halves first and the lo halves *_lo elements after them).  w3: the
 * split-f16 weights [64][terms3 * 32] as vdk_conv_desc takes them ([hi | hi]
 * for terms3 = 2, [hi | hi | lo] for 3).  Equal bit for bit to
 * vdk_res2_pair3x3 then vdk_conv2d_ex's LDS-DMA kernel over [sp0 | sp1]. */
int vdk_res2_pair3x3_conv3(const void* d_x, int x_stride, int batch, int H, int W, const void* d_w_a,
                           const float* d_b_a, const void* d_w_b, const float* d_b_b, const void* d_w3,
                           const float* d_b3, int terms3, const void* d_res, int res_stride, int res_lo, void* d_y,
                           int y_stride, int y_lo, float clamp_hi, void* stream);

/* A whole layer-1 block of ERes2Net (src/encoder_eres2net.cpp:111-137, the
 * Bottle2neck with scale 2 and 16-channel chunks, stride 1) in one launch,
 * split-f16: c = min(relu(conv1(x) + b1), clamp_hi) (1x1, ic1 -> 32, [c0 | c1])
 * then vdk_res2_pair3x3_conv3's pair and conv3 from c, with
 * res = x when d_res is NULL (ic1 = 64: the block without a shortcut conv),
 * else the given map (the shortcut output).  x: [batch][H][W] rows of
 * x_stride elements, the ic1 hi halves first and the lo halves x_lo
 * elements after them (ic1 = 32 or 64); w1: the split-f16 weights
 * [32][terms1 * ic1] as vdk_conv_desc takes them ([hi | hi] for terms1 = 2,
 * [hi | hi | lo] for 3); b1: f32 [32]; w_a, w_b, b_a, b_b, w3,
 * b3, terms3, res, y as for vdk_res2_pair3x3_conv3.  c never reaches
 * memory, so HBM sees x once and y once.  Equal bit for bit to vdk_conv2d_ex's
 * split-f16 conv1 into [c0 | c1] rows followed by vdk_res2_pair3x3_conv3.
 * y must not overlap x or res. */
int vdk_res2_bottleneck(const void* d_x, int x_stride, int x_lo, int ic1, int batch, int H, int W, const void* d_w1,
                        int terms1, const float* d_b1, const void* d_w_a, const float* d_b_a, const void* d_w_b,
                        const float* d_b_b, const void* d_w3, const float* d_b3, int terms3, const void* d_res,
                        int res_stride, int res_lo, void* d_y, int y_stride, int y_lo, float clamp_hi, void* stream);

/* ---- wav2vec2 analyze (src/analyze_w2v2.cpp) ----
 * Activations are time-major [B][T][C]; the GEMM-shaped layers run on
 * vdk_conv2d_ex (H = 1, W = T).  These cover the rest of the graph. */

/* do_normalize statistics of the raw waveform (src/analyze_w2v2.cpp:63-70):
 * stats[b] = {mean, 1/sqrt(biased var + eps)} of clip b, f64 two-pass. */
int vdk_wave_stats(const float* d_x, int batch, int n, float eps, float* d_stats, void* stream);

/* Conv layer 0 of the feature encoder (src/analyze_w2v2.cpp:34-45, 52-131):
 * one input channel, y[b][t][c] = gelu(norm(bias[c] + sum_k w[c][k] xn[b][t*S+k]))
 * with xn = (x - mean) * rstd when d_stats (vdk_wave_stats) is given, else x.
 * norm 0: none; 1: GroupNorm with one group per channel (mean / biased var of
 * each channel over the clip's T0 frames); 2: LayerNorm over the
 * C channels of each frame; affine gamma / beta, eps.  x [B][n] f32,
 * w [C][K] f32, y [B][T0][C] f16, T0 = (n - K)/S + 1, C in {256, 512, 1024},
 * K <= 16, S <= 8.  norm 1 needs vdk_w2v2_conv0_workspace_size() bytes of d_work. */
size_t vdk_w2v2_conv0_workspace_size(int batch, int n, int C, int K, int S);
int vdk_w2v2_conv0(const float* d_x, int batch, int n, const float* d_stats, const float* d_w,
                   const float* d_bias, int C, int K, int S, int norm, const float* d_gamma,
                   const float* d_beta, float eps, void* d_work, size_t work_bytes, void* d_y,
                   void* stream);

/* LayerNorm over rows of C values, biased variance (src/analyze_w2v2.cpp:187-193):
 * o = (x - mean) / sqrt(var + eps) * gamma + beta [then GELU]; y f16 or f32 (may
 * be NULL); when d_acc != NULL also acc = [acc +] acc_w * (o, or x with
 * VDK_LN_ACC_INPUT) in f32 - the emotion head's weighted layer sum
 * (src/analyze_w2v2.cpp:528-538).  C % 64 == 0, C <= 4096. */
enum { VDK_LN_X_F32 = 1, VDK_LN_Y_F32 = 2, VDK_LN_GELU = 4, VDK_LN_ACC_INPUT = 8, VDK_LN_ACC_INIT = 16 };
int vdk_layer_norm(const void* d_x, int rows, int C, const float* d_gamma, const float* d_beta, float eps,
                   int flags, void* d_y, float* d_acc, float acc_w, void* stream);

/* Multi-head self-attention core (src/analyze_w2v2.cpp:222-270): per clip and
 * head, out = softmax(q k^T * scale) v over all T tokens (no mask).
 * qkv [B][T][3H] f16 = [q | k | v] with head h at columns h*head_dim of each,
 * out [B][T][H] f16, H = n_heads * head_dim; head_dim must be 64. */
int vdk_attention(const void* d_qkv, int batch, int T, int n_heads, int head_dim, float scale,
                  void* d_out, void* stream);

/* Positional conv embedding of wav2vec2 (src/analyze_w2v2.cpp:280-326): a
 * grouped 1-D conv with kernel K and zero pad `pad` (frame t reads input frames
 * t - pad .. t - pad + K - 1; only the first T outputs are kept, as
 * Wav2Vec2SamePadLayer does for even K), its bias, GELU and the residual:
 *   y[b][t][gC+o] = x[b][t][gC+o] + gelu(bias[gC+o] + sum_k,i w[g][o][k][i] x[b][t+k-pad][gC+i])
 * x [B][T][H] f16, w [groups][64][K][C] f16 (C = H / groups in {48, 64}, output
 * rows C..63 zero), bias [H] f32, y [B][T][H] f32; K <= 128. */
int vdk_pos_conv(const void* d_x, int batch, int T, int H, int groups, const void* d_w, const float* d_bias,
                 int K, int pad, float* d_y, void* stream);

/* out[b][c] = mean over t of x[b][t][c] (f16 or f32 input, f64 sums): the
 * time mean-pool of the analyze heads (src/analyze_w2v2.cpp:546-550, 607-610). */
int vdk_time_mean(const void* d_x, int x_f32, int batch, int T, int C, float* d_out, void* stream);
/* out[b][c] = [out[b][c] +] w * mean over t of x[b][t][c] (accumulate != 0 adds):
 * the emotion head's weighted layer sum, one hidden state at a time. */
int vdk_time_mean_acc(const void* d_x, int x_f32, int batch, int T, int C, float w, int accumulate,
                      float* d_out, void* stream);

#ifdef __cplusplus
}
#endif
#endif
