// capi.cpp - the flat C ABI (include/voicedetect_capi.h, include/voicedetect_gpu.h).
//
// Same contract as the reference's src/voicedetect_capi.cpp:61-178: an owning
// opaque context holding the model and the last error; exception-free
// boundary; malloc'd outputs; outputs reset/untouched exactly as there.
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "audio.hpp"
#include "common.hpp"
#include "model.hpp"
#include "voicedetect_capi.h"
#include "voicedetect_gpu.h"

#define VOICEDETECT_CAPI_ABI_VERSION 1

struct voicedetect_ctx {
    std::unique_ptr<vdk::Model> model;
    std::string last_error;
    std::vector<vdk::ProfileRecord> profile;
    // enrolled embeddings for identify (device, [reg_n][reg_dim]) and a
    // grow-only device scratch for the identify calls
    float* reg = nullptr;
    int reg_n = 0, reg_dim = 0;
    void* scratch = nullptr;
    size_t scratch_bytes = 0;
    ~voicedetect_ctx() {
        if (model) model->synchronize();
        if (reg) (void)hipFree(reg);
        if (scratch) (void)hipFree(scratch);
    }
};

namespace {

float* dup_vec(const std::vector<float>& v) {
    if (v.empty()) return nullptr;
    float* buf = static_cast<float*>(std::malloc(v.size() * sizeof(float)));
    if (buf) std::memcpy(buf, v.data(), v.size() * sizeof(float));
    return buf;
}

int emit(voicedetect_ctx* ctx, const std::vector<float>& v, int dim, float** out_vec, int* out_dim) {
    float* buf = dup_vec(v);
    if (!buf) {
        ctx->last_error = "out of memory";
        return 1;
    }
    if (out_vec) *out_vec = buf;
    else std::free(buf);
    if (out_dim) *out_dim = dim;
    ctx->last_error.clear();
    return 0;
}

template <class F>
int run(voicedetect_ctx* ctx, F&& body) {
    try {
        return body();
    } catch (const std::exception& e) {
        ctx->last_error = e.what();
        return 1;
    } catch (...) {
        ctx->last_error = "unknown error";
        return 1;
    }
}

std::vector<float> embed_path(vdk::Model& m, const char* path) {
    std::vector<float> pcm;
    if (!vdk::load_audio_16k_mono(path, pcm))
        throw vdk::Error(std::string("voicedetect: failed to load audio: ") + path);
    return m.embed_pcm(pcm, 16000);
}

// src/model.cpp:65-78: dot in double, distance = 1 - (float)dot, verified = distance <= threshold.
void verdict(const std::vector<float>& ea, const std::vector<float>& eb, float threshold, float& distance,
             bool& verified) {
    if (ea.size() != eb.size() || ea.empty())
        throw vdk::Error("voicedetect: embedding dimension mismatch in verify");
    double dot = 0.0;
    for (size_t i = 0; i < ea.size(); ++i) dot += (double)ea[i] * (double)eb[i];
    distance = 1.0f - (float)dot;
    verified = distance <= threshold;
}

}  // namespace

extern "C" int voicedetect_capi_abi_version(void) { return VOICEDETECT_CAPI_ABI_VERSION; }

extern "C" voicedetect_ctx* voicedetect_capi_load(const char* gguf_path) {
    if (!gguf_path) return nullptr;
    try {
        std::unique_ptr<vdk::Model> m = vdk::Model::load(gguf_path);
        if (!m) return nullptr;
        auto* ctx = new (std::nothrow) voicedetect_ctx();
        if (!ctx) return nullptr;
        ctx->model = std::move(m);
        return ctx;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "[voicedetect] load failed: %s\n", e.what());
        return nullptr;
    } catch (...) {
        return nullptr;
    }
}

extern "C" void voicedetect_capi_free(voicedetect_ctx* ctx) { delete ctx; }

extern "C" const char* voicedetect_capi_last_error(voicedetect_ctx* ctx) {
    return ctx ? ctx->last_error.c_str() : "";
}

extern "C" void voicedetect_capi_free_string(char* s) { std::free(s); }

extern "C" void voicedetect_capi_free_vec(float* v) { std::free(v); }

extern "C" int voicedetect_capi_embed_path(voicedetect_ctx* ctx, const char* wav_path, float** out_vec,
                                           int* out_dim) {
    if (out_vec) *out_vec = nullptr;
    if (out_dim) *out_dim = 0;
    if (!ctx) return 1;
    if (!ctx->model) { ctx->last_error = "context has no loaded model"; return 1; }
    if (!wav_path) { ctx->last_error = "wav_path is NULL"; return 1; }
    return run(ctx, [&] {
        std::vector<float> e = embed_path(*ctx->model, wav_path);
        return emit(ctx, e, (int)e.size(), out_vec, out_dim);
    });
}

extern "C" int voicedetect_capi_embed_pcm(voicedetect_ctx* ctx, const float* pcm, int n_samples, int sample_rate,
                                          float** out_vec, int* out_dim) {
    if (out_vec) *out_vec = nullptr;
    if (out_dim) *out_dim = 0;
    if (!ctx) return 1;
    if (!ctx->model) { ctx->last_error = "context has no loaded model"; return 1; }
    if (!pcm || n_samples < 0) { ctx->last_error = "invalid pcm buffer"; return 1; }
    return run(ctx, [&] {
        std::vector<float> x(pcm, pcm + n_samples);
        std::vector<float> e = ctx->model->embed_pcm(x, sample_rate);
        return emit(ctx, e, (int)e.size(), out_vec, out_dim);
    });
}

extern "C" int voicedetect_capi_verify_paths(voicedetect_ctx* ctx, const char* a, const char* b, float threshold,
                                             float* out_distance, int* out_verified) {
    if (!ctx) return 1;
    if (!ctx->model) { ctx->last_error = "context has no loaded model"; return 1; }
    if (!a || !b) { ctx->last_error = "clip path is NULL"; return 1; }
    return run(ctx, [&] {
        const std::vector<float> ea = embed_path(*ctx->model, a);
        const std::vector<float> eb = embed_path(*ctx->model, b);
        float d = 0.0f;
        bool ok = false;
        verdict(ea, eb, threshold, d, ok);
        if (out_distance) *out_distance = d;
        if (out_verified) *out_verified = ok ? 1 : 0;
        ctx->last_error.clear();
        return 0;
    });
}

extern "C" char* voicedetect_capi_analyze_path_json(voicedetect_ctx* ctx, const char* wav_path) {
    if (!ctx) return nullptr;
    if (!ctx->model) { ctx->last_error = "context has no loaded model"; return nullptr; }
    if (!wav_path) { ctx->last_error = "wav_path is NULL"; return nullptr; }
    // src/model.cpp:80-101: analyze needs the heads and a wav2vec2 arch
    const vdk::ModelConfig& cfg = ctx->model->config();
    if (!cfg.analyze_present) {
        ctx->last_error = "voicedetect: this model has no age/gender/emotion analyze heads";
        return nullptr;
    }
    if (!ctx->model->is_analyzer()) {
        ctx->last_error = "voicedetect: analyze head unsupported for arch '" + cfg.arch + "'";
        return nullptr;
    }
    char* out = nullptr;
    run(ctx, [&] {
        std::vector<float> pcm;
        if (!vdk::load_audio_16k_mono(wav_path, pcm))
            throw vdk::Error(std::string("voicedetect: failed to load audio: ") + wav_path);
        const std::string js = ctx->model->analyze_json(pcm, 16000);
        out = static_cast<char*>(std::malloc(js.size() + 1));
        if (!out) throw vdk::Error("out of memory");
        std::memcpy(out, js.c_str(), js.size() + 1);
        ctx->last_error.clear();
        return 0;
    });
    return out;
}

extern "C" int voicedetect_capi_embedding_dim(voicedetect_ctx* ctx) {
    return (ctx && ctx->model) ? ctx->model->embedding_dim() : 0;
}

extern "C" int voicedetect_capi_embed_pcm_batch(voicedetect_ctx* ctx, const float* pcm, int batch, int n_samples,
                                                int sample_rate, float** out_vec, int* out_dim) {
    if (out_vec) *out_vec = nullptr;
    if (out_dim) *out_dim = 0;
    if (!ctx) return 1;
    if (!ctx->model) { ctx->last_error = "context has no loaded model"; return 1; }
    if (!pcm || n_samples < 0 || batch <= 0) { ctx->last_error = "invalid pcm buffer"; return 1; }
    return run(ctx, [&] {
        vdk::Model& m = *ctx->model;
        const int dim = m.embedding_dim();
        std::vector<float> out((size_t)batch * dim);
        if (sample_rate == 16000) {
            m.embed_batch_host(pcm, batch, n_samples, out.data());
        } else {
            std::vector<float> all;
            int n16 = -1;
            for (int b = 0; b < batch; ++b) {
                std::vector<float> x(pcm + (size_t)b * n_samples, pcm + (size_t)(b + 1) * n_samples);
                std::vector<float> y = vdk::resample_linear(x, sample_rate, 16000);
                n16 = (int)y.size();
                all.insert(all.end(), y.begin(), y.end());
            }
            m.embed_batch_host(all.data(), batch, n16, out.data());
        }
        return emit(ctx, out, dim, out_vec, out_dim);
    });
}

extern "C" int voicedetect_capi_verify_pcm(voicedetect_ctx* ctx, const float* a, int n_a, const float* b, int n_b,
                                           int sample_rate, float threshold, float* out_distance,
                                           int* out_verified) {
    if (!ctx) return 1;
    if (!ctx->model) { ctx->last_error = "context has no loaded model"; return 1; }
    if (!a || !b || n_a < 0 || n_b < 0) { ctx->last_error = "invalid pcm buffer"; return 1; }
    return run(ctx, [&] {
        const std::vector<float> ea = ctx->model->embed_pcm(std::vector<float>(a, a + n_a), sample_rate);
        const std::vector<float> eb = ctx->model->embed_pcm(std::vector<float>(b, b + n_b), sample_rate);
        float d = 0.0f;
        bool ok = false;
        verdict(ea, eb, threshold, d, ok);
        if (out_distance) *out_distance = d;
        if (out_verified) *out_verified = ok ? 1 : 0;
        ctx->last_error.clear();
        return 0;
    });
}

extern "C" int voicedetect_gpu_embed_batch_async(voicedetect_ctx* ctx, const float* d_pcm, int batch,
                                                 int n_samples, float* d_out) {
    if (!ctx) return 1;
    if (!ctx->model) { ctx->last_error = "context has no loaded model"; return 1; }
    return run(ctx, [&] {
        ctx->model->embed_batch_device(d_pcm, batch, n_samples, d_out);
        ctx->last_error.clear();
        return 0;
    });
}

extern "C" int voicedetect_gpu_synchronize(voicedetect_ctx* ctx) {
    if (!ctx || !ctx->model) return 1;
    return run(ctx, [&] {
        ctx->model->synchronize();
        ctx->last_error.clear();
        return 0;
    });
}

extern "C" void* voicedetect_gpu_stream(voicedetect_ctx* ctx) {
    if (!ctx || !ctx->model) return nullptr;
    void* s = nullptr;
    run(ctx, [&] {
        s = ctx->model->stream();
        return 0;
    });
    return s;
}

extern "C" int voicedetect_gpu_embed_capture(voicedetect_ctx* ctx, const float* pcm, int batch, int n_samples,
                                             float* feats, float* pooled, int* pooled_dim, float* pre_norm,
                                             float* out) {
    if (!ctx) return 1;
    if (!ctx->model) { ctx->last_error = "context has no loaded model"; return 1; }
    if (!pcm || batch <= 0 || n_samples < 0) { ctx->last_error = "invalid pcm buffer"; return 1; }
    return run(ctx, [&] {
        ctx->model->embed_capture(pcm, batch, n_samples, feats, pooled, pre_norm, out);
        if (pooled_dim) *pooled_dim = ctx->model->pooled_dim();
        ctx->last_error.clear();
        return 0;
    });
}

extern "C" int voicedetect_gpu_set_profiling(voicedetect_ctx* ctx, int on) {
    if (!ctx || !ctx->model) return 1;
    ctx->model->set_profiling(on != 0);
    return 0;
}

extern "C" int voicedetect_gpu_set_profiling_filter(voicedetect_ctx* ctx, int on, const char* name_prefix) {
    if (!ctx || !ctx->model) return 1;
    ctx->model->set_profiling(on != 0, name_prefix ? std::string(name_prefix) : std::string());
    return 0;
}

extern "C" int voicedetect_gpu_set_profiling_markers(voicedetect_ctx* ctx, int on) {
    if (!ctx || !ctx->model) return 1;
    return run(ctx, [&] {
        ctx->model->set_profiling_markers(on != 0);
        return 0;
    });
}

extern "C" int voicedetect_gpu_profile_collect(voicedetect_ctx* ctx) {
    if (!ctx || !ctx->model) return -1;
    int n = -1;
    const int rc = run(ctx, [&] {
        ctx->profile = ctx->model->take_profile();
        n = (int)ctx->profile.size();
        return 0;
    });
    return rc == 0 ? n : -1;
}

extern "C" int voicedetect_gpu_profile_get(voicedetect_ctx* ctx, int i, char* name, int name_cap, double* ms,
                                           double* flops, double* bytes) {
    if (!ctx || i < 0 || i >= (int)ctx->profile.size()) return 1;
    const vdk::ProfileRecord& r = ctx->profile[(size_t)i];
    if (name && name_cap > 0) {
        std::strncpy(name, r.name.c_str(), (size_t)name_cap - 1);
        name[name_cap - 1] = '\0';
    }
    if (ms) *ms = r.ms;
    if (flops) *flops = r.flops;
    if (bytes) *bytes = r.bytes;
    return 0;
}

namespace {

// Grows ctx->scratch to at least `bytes` (waiting for the stream before
// releasing the old block, which queued work may still use).
void* ctx_scratch(voicedetect_ctx* ctx, size_t bytes) {
    if (bytes > ctx->scratch_bytes) {
        ctx->model->synchronize();
        if (ctx->scratch) VDK_HIP(hipFree(ctx->scratch));
        ctx->scratch = nullptr;
        ctx->scratch_bytes = 0;
        VDK_HIP(hipMalloc(&ctx->scratch, bytes));
        ctx->scratch_bytes = bytes;
    }
    return ctx->scratch;
}

size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

}  // namespace

extern "C" int voicedetect_gpu_registry_set(voicedetect_ctx* ctx, const float* emb, int n, int dim) {
    if (!ctx) return 1;
    if (!ctx->model) { ctx->last_error = "context has no loaded model"; return 1; }
    if (n < 0 || (n > 0 && !emb)) { ctx->last_error = "invalid registry buffer"; return 1; }
    return run(ctx, [&] {
        vdk::require(n == 0 || dim == ctx->model->embedding_dim(),
                     "registry dim " + std::to_string(dim) + " differs from the model's embedding dim " +
                         std::to_string(ctx->model->embedding_dim()));
        ctx->model->synchronize();
        if (ctx->reg) VDK_HIP(hipFree(ctx->reg));
        ctx->reg = nullptr;
        ctx->reg_n = ctx->reg_dim = 0;
        if (n > 0) {
            VDK_HIP(hipMalloc(&ctx->reg, sizeof(float) * (size_t)n * dim));
            VDK_HIP(hipMemcpy(ctx->reg, emb, sizeof(float) * (size_t)n * dim, hipMemcpyHostToDevice));
            ctx->reg_n = n;
            ctx->reg_dim = dim;
        }
        ctx->last_error.clear();
        return 0;
    });
}

extern "C" int voicedetect_gpu_identify_device_async(voicedetect_ctx* ctx, const float* d_emb, int batch, int k,
                                                     int* d_idx, float* d_score) {
    if (!ctx) return 1;
    if (!ctx->model) { ctx->last_error = "context has no loaded model"; return 1; }
    return run(ctx, [&] {
        vdk::require(ctx->reg_n > 0, "identify: no registry (voicedetect_gpu_registry_set)");
        vdk::require(batch > 0 && d_emb && d_idx && d_score, "identify: invalid buffers");
        vdk::require(k >= 1 && k <= 64 && k <= ctx->reg_n, "identify: k must be in 1..min(64, registry size)");
        const size_t ws = vdk_registry_topk_workspace_size(batch, ctx->reg_n, k);
        void* work = ctx_scratch(ctx, ws);
        if (vdk_registry_topk(d_emb, batch, ctx->reg, ctx->reg_n, ctx->reg_dim, k, work, ws, d_idx, d_score,
                              ctx->model->stream()) != 0)
            throw vdk::Error(vdk_last_error());
        ctx->last_error.clear();
        return 0;
    });
}

extern "C" int voicedetect_gpu_identify_pcm(voicedetect_ctx* ctx, const float* pcm, int batch, int n_samples,
                                            int sample_rate, int k, int* out_idx, float* out_score) {
    if (!ctx) return 1;
    if (!ctx->model) { ctx->last_error = "context has no loaded model"; return 1; }
    if (!pcm || n_samples < 0 || batch <= 0 || !out_idx || !out_score) {
        ctx->last_error = "invalid buffers";
        return 1;
    }
    return run(ctx, [&] {
        vdk::Model& m = *ctx->model;
        vdk::require(ctx->reg_n > 0, "identify: no registry (voicedetect_gpu_registry_set)");
        vdk::require(k >= 1 && k <= 64 && k <= ctx->reg_n, "identify: k must be in 1..min(64, registry size)");
        std::vector<float> resampled;
        const float* x = pcm;
        int n16 = n_samples;
        if (sample_rate != 16000) {
            for (int b = 0; b < batch; ++b) {
                const std::vector<float> y = vdk::resample_linear(
                    std::vector<float>(pcm + (size_t)b * n_samples, pcm + (size_t)(b + 1) * n_samples), sample_rate,
                    16000);
                n16 = (int)y.size();
                resampled.insert(resampled.end(), y.begin(), y.end());
            }
            x = resampled.data();
        }
        const int dim = m.embedding_dim();
        const size_t pcm_b = align256(sizeof(float) * (size_t)batch * n16);
        const size_t emb_b = align256(sizeof(float) * (size_t)batch * dim);
        const size_t out_b = align256(sizeof(int) * (size_t)batch * k);
        const size_t ws = vdk_registry_topk_workspace_size(batch, ctx->reg_n, k);
        uint8_t* base = static_cast<uint8_t*>(ctx_scratch(ctx, pcm_b + emb_b + 2 * out_b + ws));
        float* d_pcm = reinterpret_cast<float*>(base);
        float* d_emb = reinterpret_cast<float*>(base + pcm_b);
        int* d_idx = reinterpret_cast<int*>(base + pcm_b + emb_b);
        float* d_score = reinterpret_cast<float*>(base + pcm_b + emb_b + out_b);
        void* work = base + pcm_b + emb_b + 2 * out_b;
        hipStream_t s = m.stream();
        VDK_HIP(hipMemcpyAsync(d_pcm, x, sizeof(float) * (size_t)batch * n16, hipMemcpyHostToDevice, s));
        m.embed_batch_device(d_pcm, batch, n16, d_emb);
        if (vdk_registry_topk(d_emb, batch, ctx->reg, ctx->reg_n, ctx->reg_dim, k, work, ws, d_idx, d_score, s) != 0)
            throw vdk::Error(vdk_last_error());
        VDK_HIP(hipMemcpyAsync(out_idx, d_idx, sizeof(int) * (size_t)batch * k, hipMemcpyDeviceToHost, s));
        VDK_HIP(hipMemcpyAsync(out_score, d_score, sizeof(float) * (size_t)batch * k, hipMemcpyDeviceToHost, s));
        VDK_HIP(hipStreamSynchronize(s));
        ctx->last_error.clear();
        return 0;
    });
}

extern "C" int voicedetect_gpu_analyze_outputs(voicedetect_ctx* ctx) {
    return (ctx && ctx->model) ? ctx->model->analyze_outputs() : 0;
}

extern "C" int voicedetect_gpu_analyze_frames(voicedetect_ctx* ctx, int n_samples) {
    return (ctx && ctx->model && ctx->model->is_analyzer()) ? ctx->model->analyze_frames(n_samples) : 0;
}

extern "C" int voicedetect_gpu_analyze_pcm(voicedetect_ctx* ctx, const float* pcm, int batch, int n_samples,
                                           int sample_rate, float* out_raw) {
    if (!ctx) return 1;
    if (!ctx->model) { ctx->last_error = "context has no loaded model"; return 1; }
    if (!pcm || !out_raw || batch <= 0 || n_samples <= 0) { ctx->last_error = "invalid pcm buffer"; return 1; }
    return run(ctx, [&] {
        vdk::Model& m = *ctx->model;
        if (sample_rate == 16000) {
            m.analyze_batch_host(pcm, batch, n_samples, out_raw);
        } else {
            std::vector<float> all;
            int n16 = -1;
            for (int b = 0; b < batch; ++b) {
                std::vector<float> x(pcm + (size_t)b * n_samples, pcm + (size_t)(b + 1) * n_samples);
                std::vector<float> y = vdk::resample_linear(x, sample_rate, 16000);
                n16 = (int)y.size();
                all.insert(all.end(), y.begin(), y.end());
            }
            m.analyze_batch_host(all.data(), batch, n16, out_raw);
        }
        ctx->last_error.clear();
        return 0;
    });
}

extern "C" int voicedetect_gpu_analyze_batch_async(voicedetect_ctx* ctx, const float* d_pcm, int batch,
                                                   int n_samples, float* d_raw) {
    if (!ctx) return 1;
    if (!ctx->model) { ctx->last_error = "context has no loaded model"; return 1; }
    return run(ctx, [&] {
        ctx->model->analyze_batch_device(d_pcm, batch, n_samples, d_raw);
        ctx->last_error.clear();
        return 0;
    });
}

extern "C" int voicedetect_gpu_analyze_capture(voicedetect_ctx* ctx, const float* pcm, int batch, int n_samples,
                                               float* feat, float* hidden, float* out_raw) {
    if (!ctx) return 1;
    if (!ctx->model) { ctx->last_error = "context has no loaded model"; return 1; }
    if (!pcm || batch <= 0 || n_samples <= 0) { ctx->last_error = "invalid pcm buffer"; return 1; }
    return run(ctx, [&] {
        ctx->model->analyze_capture(pcm, batch, n_samples, feat, hidden, out_raw);
        ctx->last_error.clear();
        return 0;
    });
}
