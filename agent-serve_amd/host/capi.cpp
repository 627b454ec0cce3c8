// C entry points of the host side (libtinferno.so) for harnesses that cannot link C++:
// open a GGUF as a Model over the HIP backend, run it, and write synthetic GGUFs.
// Every function returns 0 on success and a negative status on failure; the message
// is tfh_last_error(handle) (or tfh_global_error() for calls without a model).
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <exception>
#include <stdexcept>
#include <vector>
#include <string>

#include "model.hpp"
#include "synth.hpp"
#include "tokenizer.hpp"

namespace {

thread_local std::string g_err;

struct Handle {
    tfh::Model* m = nullptr;
    std::string err;
};

template <typename Fn>
int guard(Handle* h, Fn fn) {
    try {
        fn();
        return 0;
    } catch (const std::exception& e) {
        if (h) h->err = e.what();
        g_err = e.what();
        return -1;
    }
}

}  // namespace

extern "C" {

const char* tfh_global_error() { return g_err.c_str(); }
const char* tfh_last_error(void* h) { return h ? ((Handle*)h)->err.c_str() : g_err.c_str(); }

// kv_layout: -1 keeps the stage's layout, 0 seq-major, 1 head-major (main.cpp:90-91).
void* tfh_open(const char* path, const char* stage, int max_seq, int kv_layout, int device) {
    Handle* h = new Handle();
    const int rc = guard(h, [&] {
        tfh::RunConfig cfg = tfh::stage_preset(stage ? stage : "v2", 1);
        cfg.max_seq = max_seq;
        cfg.device = device;
        if (kv_layout == 0) cfg.kv_layout = tfh::KVLayout::SeqMajor;
        if (kv_layout == 1) cfg.kv_layout = tfh::KVLayout::HeadMajor;
        h->m = new tfh::Model(path, cfg);
    });
    if (rc) {
        delete h;
        return nullptr;
    }
    return h;
}

void tfh_close(void* hp) {
    Handle* h = (Handle*)hp;
    if (!h) return;
    delete h->m;
    delete h;
}

int tfh_prefill(void* hp, const int32_t* tokens, int32_t n, float* logits, int32_t* argmax) {
    Handle* h = (Handle*)hp;
    return guard(h, [&] {
        std::vector<int> t(tokens, tokens + n);
        h->m->prefill(t.data(), n, logits);
        if (argmax) *argmax = h->m->last_argmax();
    });
}

int tfh_decode(void* hp, int32_t token, float* logits, int32_t* argmax) {
    Handle* h = (Handle*)hp;
    return guard(h, [&] {
        h->m->decode(token, logits);
        if (argmax) *argmax = h->m->last_argmax();
    });
}

int tfh_generate(void* hp, int32_t n, int32_t* out) {
    Handle* h = (Handle*)hp;
    return guard(h, [&] { h->m->generate(n, out); });
}

// The greedy loop of a caller of the reference's Model with the backend switch patched in
// (bench_e2e.cpp:49-54 over model.cpp:197-208 as forwarded to tf_hip_decode): every step
// copies the logits to the host and takes their first maximum there (sample_greedy,
// sampler.cpp:8-13). out[i] is the token fed to step i, starting with `first`.
int tfh_greedy_host(void* hp, int32_t first, int32_t n, int32_t* out) {
    Handle* h = (Handle*)hp;
    return guard(h, [&] {
        std::vector<float> logits((size_t)h->m->n_vocab());
        int tok = first;
        for (int i = 0; i < n; ++i) {
            out[i] = tok;
            h->m->decode(tok, logits.data());
            tok = (int)(std::max_element(logits.begin(), logits.end()) - logits.begin());
        }
    });
}

int tfh_reset(void* hp) {
    Handle* h = (Handle*)hp;
    return guard(h, [&] { h->m->reset(); });
}

// out: vocab, embd, ff, layers, heads, kv_heads, head_dim, n_pos, max_seq, kv_layout, bos, eos
int tfh_info(void* hp, int32_t* out) {
    Handle* h = (Handle*)hp;
    return guard(h, [&] {
        const tfh::Model& m = *h->m;
        const int32_t v[12] = {m.n_vocab(), m.n_embd(), m.n_ff(), m.n_layer(), m.n_head(), m.n_kv_head(),
                               m.head_dim(), m.n_pos(), m.cfg().max_seq,
                               m.cfg().kv_layout == tfh::KVLayout::HeadMajor ? 1 : 0, m.bos(), m.eos()};
        std::memcpy(out, v, sizeof v);
    });
}

uint64_t tfh_weight_bytes(void* hp) { return hp ? (uint64_t)((Handle*)hp)->m->weight_bytes() : 0; }
double tfh_decode_bytes(void* hp, int32_t pos) { return hp ? ((Handle*)hp)->m->decode_bytes(pos) : 0.0; }

int tfh_layer_act(void* hp, int32_t layer, float* out) {
    Handle* h = (Handle*)hp;
    return guard(h, [&] {
        if (tf_hip_get_layer_act(h->m->ctx(), layer, out) != 0) throw std::runtime_error(tf_hip_last_error(h->m->ctx()));
    });
}

int tfh_read_kv(void* hp, int32_t layer, int32_t which, int32_t pos0, int32_t n, float* out) {
    Handle* h = (Handle*)hp;
    return guard(h, [&] {
        if (tf_hip_read_kv(h->m->ctx(), layer, which, pos0, n, out) != 0)
            throw std::runtime_error("read_kv: bad arguments");
    });
}

void* tfh_ctx(void* hp) { return hp ? (void*)((Handle*)hp)->m->ctx() : nullptr; }

int tfh_synth_write(const char* preset, const char* path, int64_t seed, int32_t threads, uint64_t* weight_bytes) {
    return guard(nullptr, [&] {
        tfh::SynthSpec s;
        if (!tfh::synth_preset(preset, &s)) throw std::runtime_error(std::string("unknown preset ") + preset);
        if (seed >= 0) s.seed = (uint64_t)seed;
        const uint64_t wb = tfh::synth_write(s, path, threads);
        if (weight_bytes) *weight_bytes = wb;
    });
}

// out: vocab, embd, ff, layers, heads, kv_heads, seed
int tfh_synth_preset_info(const char* preset, int32_t* out) {
    return guard(nullptr, [&] {
        tfh::SynthSpec s;
        if (!tfh::synth_preset(preset, &s)) throw std::runtime_error(std::string("unknown preset ") + preset);
        const int32_t v[7] = {s.n_vocab, s.n_embd, s.n_ff, s.n_layer, s.n_head, s.n_kv_head, (int32_t)s.seed};
        std::memcpy(out, v, sizeof v);
    });
}

int tfh_synth_prompt(int64_t seed, int32_t n, int32_t n_vocab, int32_t* out) {
    return guard(nullptr, [&] {
        const auto ids = tfh::synth_prompt((uint64_t)seed, n, n_vocab);
        std::memcpy(out, ids.data(), ids.size() * sizeof(int32_t));
    });
}

// The writer's block quantizers (one row of n elements of a ggml type).
int tfh_quantize_row(int32_t ggml_type, const float* x, int64_t n, uint8_t* out) {
    return guard(nullptr, [&] { tfh::quantize_row(ggml_type, x, n, out); });
}

// Summary of a GGUF file as the host reader sees it: out = n_tensors, weight_bytes, file_size.
int tfh_gguf_summary(const char* path, uint64_t* out, char* arch, int32_t arch_len) {
    return guard(nullptr, [&] {
        tfh::GgufFile g(path);
        out[0] = g.tensors().size();
        out[1] = g.weight_bytes();
        out[2] = g.file_size();
        if (arch && arch_len > 0) std::snprintf(arch, (size_t)arch_len, "%s", g.arch().c_str());
    });
}

// Model::decode_bytes(pos) of the GGUF at path, without a device: the algorithmic bytes of
// one decode step at position pos.
double tfh_file_decode_bytes(const char* path, int32_t pos) {
    double v = -1.0;
    guard(nullptr, [&] {
        tfh::GgufFile g(path);
        v = tfh::decode_traffic(g, tfh::read_hparams(g)).at(pos);
    });
    return v;
}

// The host RoPE tables of the GGUF at path (the Model's hyperparameter rules, llama3
// scaling included): [n_pos][head_dim / 2] cosines and sines.
int tfh_file_rope_tables(const char* path, int32_t n_pos, float* cos_out, float* sin_out) {
    return guard(nullptr, [&] {
        tfh::GgufFile g(path);
        const tfh::HParams h = tfh::read_hparams(g);
        std::vector<float> c, s;
        tfh::rope_tables(tfh::rope_freqs(h.rope), n_pos, c, s);
        std::memcpy(cos_out, c.data(), c.size() * 4);
        std::memcpy(sin_out, s.data(), s.size() * 4);
    });
}

int tfh_rope_tables(float theta, int32_t n_rot, int32_t n_pos, float* cos_out, float* sin_out) {
    return guard(nullptr, [&] {
        tfh::RopeParams rp;
        rp.theta = theta;
        rp.n_rot = n_rot;
        std::vector<float> c, s;
        tfh::rope_tables(tfh::rope_freqs(rp), n_pos, c, s);
        std::memcpy(cos_out, c.data(), c.size() * 4);
        std::memcpy(sin_out, s.data(), s.size() * 4);
    });
}

// Tokenizer::encode (tokenizer.cpp:183-201) of text with the vocabulary of the GGUF at
// path: writes up to cap ids to out and returns how many the text has (or < 0).
int32_t tfh_tokenize_file(const char* path, const char* text, int32_t add_bos, int32_t* out, int32_t cap) {
    int32_t n = -1;
    guard(nullptr, [&] {
        tfh::GgufFile g(path);
        const tfh::Tokenizer tok(g);
        const std::vector<int> ids = tok.encode(text, add_bos != 0);
        for (size_t i = 0; i < ids.size() && (int32_t)i < cap; ++i) out[i] = ids[i];
        n = (int32_t)ids.size();
    });
    return n;
}

// Tokenizer::decode (tokenizer.cpp:233-237) of ids with the vocabulary of the GGUF at path:
// writes the bytes (up to cap) to out and returns their count (or < 0).
int32_t tfh_detokenize_file(const char* path, const int32_t* ids, int32_t n, char* out, int32_t cap) {
    int32_t len = -1;
    guard(nullptr, [&] {
        tfh::GgufFile g(path);
        const tfh::Tokenizer tok(g);
        const std::string s = tok.decode(std::vector<int>(ids, ids + n));
        std::memcpy(out, s.data(), std::min(s.size(), (size_t)std::max(cap, 0)));
        len = (int32_t)s.size();
    });
    return len;
}

}  // extern "C"
