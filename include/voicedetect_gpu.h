/*
 * voicedetect_gpu.h - device-resident entry points of the MI355X library.
 *
 * For callers that keep PCM and embeddings in HBM (serving loops, batch
 * pipelines).  No counterpart in the reference, whose ABI is host-only and one
 * clip per call (reference include/voicedetect_capi.h:59-67); these add the
 * batched device path over the same context.  Same status convention as the
 * C ABI: 0 = success, nonzero = error with voicedetect_capi_last_error(ctx).
 */
#ifndef VOICEDETECT_GPU_H
#define VOICEDETECT_GPU_H

#include "voicedetect_capi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Enqueue the whole path for `batch` clips of n_samples 16 kHz f32 PCM at
 * d_pcm (device, clip-major) writing batch x dim f32 embeddings to d_out
 * (device) on the context's stream.  Returns once enqueued. */
int voicedetect_gpu_embed_batch_async(voicedetect_ctx* ctx, const float* d_pcm,
                                      int batch, int n_samples, float* d_out);

/* Wait for the context's stream. */
int voicedetect_gpu_synchronize(voicedetect_ctx* ctx);

/* The context's hipStream_t (initialises the device on first use); NULL on error. */
void* voicedetect_gpu_stream(voicedetect_ctx* ctx);

/* Host-buffer embed that also returns intermediates (any output may be NULL):
 * feats [batch][n_mels][T], pooled [batch][pooled_dim], pre_norm / out [batch][dim].
 * *pooled_dim receives the pooled width when not NULL. */
int voicedetect_gpu_embed_capture(voicedetect_ctx* ctx, const float* pcm, int batch,
                                  int n_samples, float* feats, float* pooled,
                                  int* pooled_dim, float* pre_norm, float* out);

/* Per-launch timing with HIP events recorded on the context's stream. */
int voicedetect_gpu_set_profiling(voicedetect_ctx* ctx, int on);
/* Same, recording only launches whose name starts with name_prefix (NULL or
 * "": all), so one kernel can be timed with few events in the stream. */
int voicedetect_gpu_set_profiling_filter(voicedetect_ctx* ctx, int on, const char* name_prefix);
/* While profiling, bracket every recorded launch with a one-thread marker
 * dispatch (kernel profile_marker_kernel storing 1 before, 2 after), so a
 * hardware-counter run that lists dispatches in order can attribute each
 * dispatch to its record. No counterpart in the reference (a measurement aid). */
int voicedetect_gpu_set_profiling_markers(voicedetect_ctx* ctx, int on);
/* Waits, then returns the number of launch records collected since the last
 * read (or -1 on error); records are read with voicedetect_gpu_profile_get. */
int voicedetect_gpu_profile_collect(voicedetect_ctx* ctx);
int voicedetect_gpu_profile_get(voicedetect_ctx* ctx, int i, char* name, int name_cap,
                                double* ms, double* flops, double* bytes);

/* ---- identify: score clips against an enrolled registry ----
 * No counterpart in the reference's code (README.md:15 promises identify; no
 * function or ABI symbol provides it); scores follow its verify
 * (src/model.cpp:65-78): score = sum(e_query * e_enrolled) with exact f32
 * products summed in f64, i.e. 1 - verify's distance; top k rows per clip,
 * highest score first, equal scores by the lower row. */

/* Copy n enrolled embeddings (host f32 [n][dim], dim = the model's embedding
 * dim) into HBM, replacing the previous registry; n = 0 clears it. */
int voicedetect_gpu_registry_set(voicedetect_ctx* ctx, const float* emb, int n, int dim);

/* Embed `batch` clips of host PCM on the GPU and return each clip's k best
 * registry rows (1 <= k <= min(64, n)): out_idx / out_score [batch][k] (host). */
int voicedetect_gpu_identify_pcm(voicedetect_ctx* ctx, const float* pcm, int batch, int n_samples,
                                 int sample_rate, int k, int* out_idx, float* out_score);

/* Same for device-resident embeddings d_emb [batch][dim]; writes d_idx /
 * d_score [batch][k] (device) on the context's stream and returns once
 * enqueued (the scratch it needs is allocated on first use). */
int voicedetect_gpu_identify_device_async(voicedetect_ctx* ctx, const float* d_emb, int batch, int k,
                                          int* d_idx, float* d_score);

/* ---- analyze: the wav2vec2 emotion / age-gender heads ----
 * Batched counterparts of voicedetect_capi_analyze_path_json for a context
 * loaded from an analyze GGUF (arch wav2vec2_emotion / wav2vec2_age_gender;
 * reference src/analyze_w2v2.cpp:503-558 emotion_logits, :596-630
 * age_gender_raw).  Raw outputs per clip: the emotion logits, or
 * [age_raw, gender logits...] (age in years = 100 * age_raw; probabilities are
 * the softmax of the logits). */

/* Raw outputs per clip (0 for a speaker-embedding model). */
int voicedetect_gpu_analyze_outputs(voicedetect_ctx* ctx);
/* Frames T' after the conv feature encoder for n_samples (0 if too short). */
int voicedetect_gpu_analyze_frames(voicedetect_ctx* ctx, int n_samples);

/* `batch` clips of host PCM -> out_raw [batch][outputs] (host). */
int voicedetect_gpu_analyze_pcm(voicedetect_ctx* ctx, const float* pcm, int batch, int n_samples,
                                int sample_rate, float* out_raw);

/* Device-resident batch of 16 kHz PCM d_pcm [batch][n_samples] -> d_raw
 * [batch][outputs] on the context's stream; returns once enqueued. */
int voicedetect_gpu_analyze_batch_async(voicedetect_ctx* ctx, const float* d_pcm, int batch,
                                        int n_samples, float* d_raw);

/* Host-buffer analyze that also returns intermediates (any may be NULL):
 * feat [batch][T'][conv_dim] (the conv feature encoder output, time-major),
 * hidden [batch][T'][hidden] (the last hidden state of the transformer stack),
 * out_raw [batch][outputs]. */
int voicedetect_gpu_analyze_capture(voicedetect_ctx* ctx, const float* pcm, int batch, int n_samples,
                                    float* feat, float* hidden, float* out_raw);

#ifdef __cplusplus
}
#endif

#endif
