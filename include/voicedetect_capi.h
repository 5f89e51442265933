/*
 * voicedetect_capi.h - flat C ABI of the MI355X speaker-embedding library.
 *
 * The first ten functions are the reference's frozen ABI v1, with the same
 * names, signatures, ownership and error contract
 * (reference include/voicedetect_capi.h:31-89, src/voicedetect_capi.cpp:61-178):
 * a GGUF model is loaded once into an opaque context; no C++ exception crosses
 * the boundary; failures return nonzero (or NULL) and leave a message in
 * voicedetect_capi_last_error(ctx); vectors and strings handed out are
 * malloc'd and released with voicedetect_capi_free_vec / _free_string.
 *
 * The path behind it runs entirely on one MI355X: Kaldi FBank -> speaker
 * encoder convolutions -> statistics pooling -> FC -> L2 norm.  The GGUF is
 * parsed at load; the GPU is initialised and the weights uploaded on the first
 * embed call.  A context must not be used by two threads at the same time.
 *
 * The functions after the frozen block are additive (no ABI bump, as the
 * reference's versioning rule allows).
 */
#ifndef VOICEDETECT_CAPI_H
#define VOICEDETECT_CAPI_H

#ifdef __cplusplus
extern "C" {
#endif

typedef struct voicedetect_ctx voicedetect_ctx;

/* ---------------- frozen ABI v1 ---------------- */

/* Returns 1 (reference voicedetect_capi.cpp:18,61-63). */
int voicedetect_capi_abi_version(void);

/* Loads a GGUF speaker model; NULL on a missing/bad file (reference :65-78). */
voicedetect_ctx* voicedetect_capi_load(const char* gguf_path);

/* Releases a context; NULL is ignored (reference :80-82). */
void voicedetect_capi_free(voicedetect_ctx* ctx);

/* Last error message on ctx, "" if none or if ctx is NULL (reference :84-87). */
const char* voicedetect_capi_last_error(voicedetect_ctx* ctx);

/* free() for strings / vectors returned by this library; NULL-safe (reference :89-95). */
void voicedetect_capi_free_string(char* s);
void voicedetect_capi_free_vec(float* v);

/* Embedding of a WAV file (decoded, averaged to mono, resampled to 16 kHz).
 * 0 on success with *out_vec = malloc'd *out_dim floats; nonzero on error with
 * *out_vec = NULL, *out_dim = 0 (reference :97-114). */
int voicedetect_capi_embed_path(voicedetect_ctx* ctx, const char* wav_path,
                                float** out_vec, int* out_dim);

/* Embedding of mono float PCM; resampled linearly when sample_rate != 16000
 * (reference :116-135). */
int voicedetect_capi_embed_pcm(voicedetect_ctx* ctx, const float* pcm,
                               int n_samples, int sample_rate,
                               float** out_vec, int* out_dim);

/* Cosine distance 1 - <e_a, e_b> of two WAV clips and verdict distance <= threshold.
 * Outputs untouched on error (reference :137-158, src/model.cpp:65-78). */
int voicedetect_capi_verify_paths(voicedetect_ctx* ctx, const char* a,
                                  const char* b, float threshold,
                                  float* out_distance, int* out_verified);

/* Age/gender/emotion analysis of a WAV file as a malloc'd JSON string (free
 * with voicedetect_capi_free_string), for a context loaded from a wav2vec2
 * analyze GGUF (arch wav2vec2_emotion / wav2vec2_age_gender), run on the GPU
 * (reference :160-178, src/model.cpp:80-101, src/analyze_w2v2.cpp).  On a
 * speaker-embedding model: NULL with the reference's error text
 * "voicedetect: this model has no age/gender/emotion analyze heads". */
char* voicedetect_capi_analyze_path_json(voicedetect_ctx* ctx,
                                         const char* wav_path);

/* ---------------- additive ---------------- */

/* Embedding dimension of the loaded model (0 if ctx is NULL). */
int voicedetect_capi_embedding_dim(voicedetect_ctx* ctx);

/* Batched embedding of `batch` clips of `n_samples` each, laid out clip-major
 * in `pcm`.  On success *out_vec = malloc'd batch * *out_dim floats (clip b's
 * embedding at b * *out_dim).  Error contract as embed_pcm. */
int voicedetect_capi_embed_pcm_batch(voicedetect_ctx* ctx, const float* pcm,
                                     int batch, int n_samples, int sample_rate,
                                     float** out_vec, int* out_dim);

/* Verify from in-memory PCM (same rule as verify_paths, no file I/O). */
int voicedetect_capi_verify_pcm(voicedetect_ctx* ctx,
                                const float* a, int n_a, const float* b, int n_b,
                                int sample_rate, float threshold,
                                float* out_distance, int* out_verified);

#ifdef __cplusplus
}
#endif

#endif
