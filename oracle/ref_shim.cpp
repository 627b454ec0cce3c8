// ref_shim.cpp - C entry points over the reference library compiled from its own sources.
//
// TEST INFRASTRUCTURE ONLY. oracle/Makefile compiles the reference's src/*.cpp with
// the reference's flags into oracle/_ref/ and links this shim beside them, so that the
// tests can pin the oracle (oracle.c) against the real reference bit for bit, and so
// that bench.py can time the reference --stage v2 path as the CPU baseline. Nothing
// in the product loads it.
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <exception>
#include <string>
#include <thread>
#include <random>
#include <vector>

#include "attention.hpp"
#include "layers.hpp"
#include "matmul.hpp"
#include "model.hpp"
#include "quant.hpp"
#include "sampler.hpp"
#include "tokenizer.hpp"

using namespace tinf;

namespace {

thread_local std::string g_err;

Tensor view(int type, const void* data, int64_t rows, int64_t cols) {
    Tensor t;
    t.dtype = dtype_from_ggml(type);
    t.ndim = 2;
    t.shape[0] = cols;
    t.shape[1] = rows;
    t.data = (const uint8_t*)data;
    t.nbytes = (size_t)rows * row_nbytes(t.dtype, cols);
    return t;
}

}  // namespace

extern "C" {

const char* ref_last_error() { return g_err.c_str(); }

float ref_f16_to_f32(uint16_t h) { return f16_to_f32(h); }

int ref_dequant_row(int type, const void* row, int64_t n, float* out) {
    try {
        Tensor t = view(type, row, 1, n);
        dequant_row(out, t, 0);
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

// C[M,N] = A[M,K] W[N,K]^T through tinf::matmul with the v2 preset (matmul.cpp:64-73).
int ref_matmul(float* c, const float* a, int m, int type, const void* w, int64_t n, int64_t k, int threads) {
    try {
        RunConfig cfg = stage_preset("v2", threads > 0 ? threads : 1);
        ThreadPool pool(cfg.n_threads, false);
        Exec ex{&cfg, &pool, nullptr};
        Tensor t = view(type, w, n, k);
        matmul(c, a, t, m, ex);
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

float ref_dot_f32(const float* a, const float* b, int n) { return dot_f32(a, b, n, true); }

void ref_rmsnorm(float* out, const float* x, const float* w, int n, float eps) { rmsnorm(out, x, w, n, eps); }
void ref_silu_mul(float* g, const float* u, int n) { silu_mul(g, u, n); }
void ref_softmax(float* x, int n) { softmax(x, n); }
int ref_argmax(const float* x, int n) { return sample_greedy(x, n); }

// The reference's sampling loop (main.cpp:109-116): one std::mt19937(seed), then n_draws
// calls of sample_logits on the same logits.
void ref_sample_logits_seq(const float* logits, int n, float temperature, float top_p, uint32_t seed, int n_draws,
                           int32_t* out) {
    std::mt19937 rng(seed);
    for (int i = 0; i < n_draws; ++i) out[i] = sample_logits(logits, n, temperature, top_p, rng);
}

// Tokenizer::encode / decode of the reference over the GGUF at path (ids up to cap; returns
// the full count, or -1 with ref_last_error()).
int32_t ref_tokenize(const char* path, const char* text, int32_t add_bos, int32_t* out, int32_t cap) {
    try {
        GGUF g(path);
        Tokenizer tok(g);
        const std::vector<int> ids = tok.encode(text, add_bos != 0);
        for (size_t i = 0; i < ids.size() && (int32_t)i < cap; ++i) out[i] = ids[i];
        return (int32_t)ids.size();
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

int32_t ref_detokenize(const char* path, const int32_t* ids, int32_t n, char* out, int32_t cap) {
    try {
        GGUF g(path);
        Tokenizer tok(g);
        const std::string s = tok.decode(std::vector<int>(ids, ids + n));
        std::memcpy(out, s.data(), std::min(s.size(), (size_t)(cap > 0 ? cap : 0)));
        return (int32_t)s.size();
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

// The uniform draws sample_logits makes (sampler.cpp:44-45) from std::mt19937(seed).
void ref_uniform_draws(uint32_t seed, int n, float* out) {
    std::mt19937 rng(seed);
    std::uniform_real_distribution<float> dist(0.0f, 1.0f);
    for (int i = 0; i < n; ++i) out[i] = dist(rng);
}

void ref_rope_freqs(float* freq, int n_rot, float theta, int llama3, float scale, float lo, float hi, float orig) {
    RopeParams rp;
    rp.type = llama3 ? RopeType::Llama3 : RopeType::Standard;
    rp.theta = theta;
    rp.n_rot = n_rot;
    rp.scale = scale;
    rp.low_freq_f = lo;
    rp.high_freq_f = hi;
    rp.orig_ctx = orig;
    std::vector<float> f;
    rope_freqs(f, rp);
    std::memcpy(freq, f.data(), f.size() * sizeof(float));
}

void ref_rope(float* x, int n_heads, int head_dim, int pos, const float* freq) {
    apply_rope(x, n_heads, head_dim, pos, freq, nullptr);
}

// k, v: logical rows [n_pos][n_kv][hd]; they are stored into a one-layer KVCache of the
// given layout (kvcache.cpp:31-36) before attn_decode (attention.cpp:55-80) reads them.
void ref_attn_decode(float* out, const float* q, const float* k, const float* v, int layout, int n_kv,
                     int max_seq, int n_heads, int hd, int n_pos) {
    KVCache kv;
    kv.init(1, n_kv, hd, max_seq, layout ? KVLayout::HeadMajor : KVLayout::SeqMajor);
    for (int p = 0; p < n_pos; ++p) kv.store(0, p, k + (size_t)p * n_kv * hd, v + (size_t)p * n_kv * hd);
    std::vector<float> scores((size_t)max_seq + 1);
    attn_decode(out, q, kv, 0, n_heads, n_kv, hd, n_pos, scores.data(), nullptr);
}

void ref_attn_prefill(float* out, const float* q, const float* k, const float* v, int seq, int n_heads,
                      int n_kv, int hd) {
    std::vector<float> scores((size_t)seq + 1);
    attn_prefill(out, q, k, v, seq, n_heads, n_kv, hd, scores.data(), nullptr);
}

// Model(path, stage_preset(stage)) with the CLI's overrides (main.cpp:79-91).
void* ref_open(const char* path, const char* stage, int max_seq, int kv_layout, int threads) {
    try {
        int hw = (int)std::thread::hardware_concurrency();
        if (hw <= 0) hw = 4;
        RunConfig cfg = stage_preset(stage, hw);
        if (threads > 0) cfg.n_threads = threads;
        cfg.max_seq = max_seq;
        if (kv_layout == 0) cfg.kv_layout = KVLayout::SeqMajor;
        if (kv_layout == 1) cfg.kv_layout = KVLayout::HeadMajor;
        return new Model(path, cfg);
    } catch (const std::exception& e) {
        g_err = e.what();
        return nullptr;
    }
}

void ref_close(void* m) { delete (Model*)m; }

int ref_prefill(void* m, const int32_t* tokens, int n, float* logits) {
    try {
        std::vector<int> t(tokens, tokens + n);
        ((Model*)m)->prefill(t.data(), n, logits);
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

int ref_decode(void* m, int32_t token, float* logits) {
    try {
        ((Model*)m)->decode(token, logits);
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

void ref_reset(void* m) { ((Model*)m)->reset(); }

// out: vocab, embd, layers, n_pos, bos, eos, threads
void ref_info(void* mp, int32_t* out) {
    Model* m = (Model*)mp;
    out[0] = m->n_vocab();
    out[1] = m->n_embd();
    out[2] = m->n_layer();
    out[3] = m->n_pos();
    out[4] = m->bos();
    out[5] = m->eos();
    out[6] = m->cfg().n_threads;
}

uint64_t ref_weight_bytes(void* m) { return (uint64_t)((Model*)m)->weight_bytes(); }

// The bench_e2e timing loop (bench_e2e.cpp:38-59): reset, prefill, then n greedy decode steps
// (sample_greedy + decode each). Writes the generated ids and the wall-clock seconds of both parts.
int ref_generate(void* mp, const int32_t* prompt, int n_prompt, int n_predict, int32_t* out_ids,
                 double* prefill_s, double* decode_s) {
    try {
        Model* m = (Model*)mp;
        m->reset();
        std::vector<int> p(prompt, prompt + n_prompt);
        std::vector<float> logits((size_t)m->n_vocab());
        double t0 = now_s();
        m->prefill(p.data(), n_prompt, logits.data());
        *prefill_s = now_s() - t0;
        t0 = now_s();
        for (int i = 0; i < n_predict; ++i) {
            const int id = sample_greedy(logits.data(), m->n_vocab());
            out_ids[i] = id;
            m->decode(id, logits.data());
        }
        *decode_s = now_s() - t0;
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

}  // extern "C"
