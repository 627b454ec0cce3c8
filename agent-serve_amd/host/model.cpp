#include "model.hpp"

#include <cmath>
#include <sstream>
#include <stdexcept>

namespace tfh {

RunConfig stage_preset(const std::string& stage, int hw_threads) {
    RunConfig c;
    c.stage = stage;
    const int nt = hw_threads > 1 ? hw_threads : 1;
    if (stage == "v0") {
        c.n_threads = 1;
    } else if (stage == "v1") {
        c.n_threads = nt;
    } else if (stage == "v2" || stage == "v3") {
        c.n_threads = nt;
        c.use_simd = true;
    } else if (stage == "v4") {
        c.n_threads = nt;
        c.use_simd = true;
        c.use_blocking = true;
    } else if (stage == "v5") {
        c.n_threads = nt;
        c.use_simd = true;
        c.use_blocking = true;
        c.kv_layout = KVLayout::HeadMajor;
    } else {
        throw std::runtime_error("unknown stage " + stage + " (use v0..v5)");
    }
    return c;
}

std::vector<float> rope_freqs(const RopeParams& rp) {
    const int d2 = rp.n_rot / 2;
    std::vector<float> freq((size_t)d2);
    for (int i = 0; i < d2; ++i) {
        float f = 1.0f / std::pow(rp.theta, (float)(2 * i) / (float)rp.n_rot);
        if (rp.llama3) {
            const float wavelen = 2.0f * 3.14159265358979323846f / f;
            const float lo_wl = rp.orig_ctx / rp.low_freq_f;
            const float hi_wl = rp.orig_ctx / rp.high_freq_f;
            if (wavelen < hi_wl) {
            } else if (wavelen > lo_wl) {
                f /= rp.scale;
            } else {
                const float smooth = (rp.orig_ctx / wavelen - rp.low_freq_f) / (rp.high_freq_f - rp.low_freq_f);
                // the reference's -mfma build fuses smooth * f into the sum
                f = std::fma(smooth, f, (1.0f - smooth) * f / rp.scale);
            }
        }
        freq[(size_t)i] = f;
    }
    return freq;
}

void rope_tables(const std::vector<float>& freq, int n_pos, std::vector<float>& ct, std::vector<float>& st) {
    const size_t d2 = freq.size();
    ct.resize((size_t)n_pos * d2);
    st.resize((size_t)n_pos * d2);
    for (int p = 0; p < n_pos; ++p)
        for (size_t i = 0; i < d2; ++i) {
            const float ang = (float)p * freq[i];
            ct[(size_t)p * d2 + i] = std::cos(ang);
            st[(size_t)p * d2 + i] = std::sin(ang);
        }
}

void Model::check(int rc, const char* what) const {
    if (rc != 0) {
        std::string msg = ctx_ ? tf_hip_last_error(ctx_) : "";
        if (msg.empty()) msg = std::string(what) + " failed (status " + std::to_string(rc) + ")";
        throw std::runtime_error(msg);
    }
}

namespace {

const char* const kLayerNames[TF_HIP_LAYER_COUNT] = {
    "attn_norm.weight", "attn_q.weight",   "attn_k.weight", "attn_v.weight",   "attn_output.weight",
    "attn_q.bias",      "attn_k.bias",     "attn_v.bias",   "ffn_norm.weight", "ffn_gate.weight",
    "ffn_up.weight",    "ffn_down.weight"};

bool optional_kind(int k) { return k == TF_HIP_LAYER_BQ || k == TF_HIP_LAYER_BK || k == TF_HIP_LAYER_BV; }

}  // namespace

HParams read_hparams(const GgufFile& g) {
    HParams h;
    const std::string a = g.arch();
    auto key = [&](const char* f) { return a + "." + f; };
    h.n_vocab = (int)g.u64(key("vocab_size"), 0);
    if (!h.n_vocab) h.n_vocab = (int)g.arr_len("tokenizer.ggml.tokens");
    h.n_embd = (int)g.u64(key("embedding_length"));
    h.n_ff = (int)g.u64(key("feed_forward_length"));
    h.n_layer = (int)g.u64(key("block_count"));
    h.n_head = (int)g.u64(key("attention.head_count"));
    h.n_kv_head = (int)g.u64(key("attention.head_count_kv"), (uint64_t)h.n_head);
    h.head_dim = h.n_head ? h.n_embd / h.n_head : 0;  // n_embd / n_head wins over rope.dimension_count
    h.rms_eps = g.f32(key("attention.layer_norm_rms_epsilon"), 1e-5f);
    RopeParams& rp = h.rope;
    rp.theta = g.f32(key("rope.freq_base"), 10000.0f);
    rp.n_rot = h.head_dim;
    if (g.str(key("rope.scaling.type"), "") == "llama3") {
        rp.llama3 = true;
        rp.scale = g.f32(key("rope.scaling.factor"), 32.0f);
        rp.low_freq_f = g.f32(key("rope.scaling.low_freq_factor"), 1.0f);
        rp.high_freq_f = g.f32(key("rope.scaling.high_freq_factor"), 4.0f);
        rp.orig_ctx = (float)g.u64(key("rope.scaling.original_context_length"), 8192);
    }
    h.bos = (int)g.u64("tokenizer.ggml.bos_token_id", 1);
    h.eos = (int)g.u64("tokenizer.ggml.eos_token_id", 2);
    if (!h.n_vocab) h.n_vocab = (int)g.must("token_embd.weight").rows();
    if (h.n_layer <= 0 || h.n_embd <= 0 || h.n_head <= 0) throw std::runtime_error("bad hyperparameters");
    return h;
}

DecodeTraffic decode_traffic(const GgufFile& g, const HParams& hp) {
    DecodeTraffic t;
    const TensorInfo& tok = g.must("token_embd.weight");
    const TensorInfo* out = g.find("output.weight");
    // tied: token_embd is the lm_head and read whole; untied: output is, and one row of token_embd
    t.tensor_bytes = out ? out->nbytes : tok.nbytes;
    t.tensor_bytes += g.must("output_norm.weight").nbytes;
    for (int l = 0; l < hp.n_layer; ++l)
        for (int k = 0; k < TF_HIP_LAYER_COUNT; ++k) {
            const std::string name = "blk." + std::to_string(l) + "." + kLayerNames[k];
            const TensorInfo* ti = optional_kind(k) ? g.find(name) : &g.must(name);
            if (ti) t.tensor_bytes += ti->nbytes;
        }
    t.embd_row_bytes = ggml_row_nbytes(tok.type, tok.ne[0]);
    t.kv_bytes_per_pos = (double)hp.n_layer * hp.n_kv_head * hp.head_dim * 4.0 * 2.0;
    return t;
}

Model::Model(const std::string& path, const RunConfig& cfg) : gguf_(path), cfg_(cfg) {
    const HParams h = read_hparams(gguf_);
    n_vocab_ = h.n_vocab;
    n_embd_ = h.n_embd;
    n_ff_ = h.n_ff;
    n_layer_ = h.n_layer;
    n_head_ = h.n_head;
    n_kv_head_ = h.n_kv_head;
    head_dim_ = h.head_dim;
    rms_eps_ = h.rms_eps;
    bos_ = h.bos;
    eos_ = h.eos;
    traffic_ = decode_traffic(gguf_, h);

    const TensorInfo& tok = gguf_.must("token_embd.weight");
    const TensorInfo& onorm = gguf_.must("output_norm.weight");
    const TensorInfo* out = gguf_.find("output.weight");

    tf_hip_hparams hp{};
    hp.n_vocab = n_vocab_;
    hp.n_embd = n_embd_;
    hp.n_ff = n_ff_;
    hp.n_layer = n_layer_;
    hp.n_head = n_head_;
    hp.n_kv_head = n_kv_head_;
    hp.head_dim = head_dim_;
    hp.max_seq = cfg_.max_seq;
    hp.kv_layout = cfg_.kv_layout == KVLayout::HeadMajor ? TF_HIP_KV_HEAD_MAJOR : TF_HIP_KV_SEQ_MAJOR;
    hp.rms_eps = rms_eps_;
    int rc = tf_hip_create(cfg_.device, &hp, &ctx_);
    if (rc != 0) throw std::runtime_error("tf_hip_create failed (status " + std::to_string(rc) + ")");

    auto up = [&](int slot, const TensorInfo& t) {
        check(tf_hip_upload_tensor(ctx_, slot, t.type, t.ne[0], t.rows(), t.data, t.nbytes), t.name.c_str());
    };
    up(TF_HIP_SLOT_TOKEN_EMBD, tok);
    up(TF_HIP_SLOT_OUTPUT_NORM, onorm);
    if (out) up(TF_HIP_SLOT_OUTPUT, *out);
    for (int l = 0; l < n_layer_; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        for (int k = 0; k < TF_HIP_LAYER_COUNT; ++k) {
            const TensorInfo* t = optional_kind(k) ? gguf_.find(p + kLayerNames[k]) : &gguf_.must(p + kLayerNames[k]);
            if (t) up(TF_HIP_SLOT_LAYER(l, k), *t);
        }
    }
    std::vector<float> ct, st;
    rope_tables(rope_freqs(h.rope), cfg_.max_seq, ct, st);
    check(tf_hip_set_rope_table(ctx_, ct.data(), st.data(), cfg_.max_seq, head_dim_ / 2), "rope table");
}

Model::~Model() { tf_hip_destroy(ctx_); }

void Model::prefill(const int* tokens, int n, float* logits) {
    if (n <= 0) return;
    if (n > cfg_.max_seq - n_pos_) throw std::runtime_error("prefill exceeds max_seq");
    std::vector<int32_t> t(tokens, tokens + n);
    int32_t am = -1;
    check(tf_hip_prefill(ctx_, t.data(), n, logits, &am), "prefill");
    last_argmax_ = am;
    n_pos_ += n;
}

void Model::decode(int token, float* logits) {
    if (n_pos_ >= cfg_.max_seq) throw std::runtime_error("decode exceeds max_seq");
    int32_t am = -1;
    check(tf_hip_decode(ctx_, token, logits, &am), "decode");
    last_argmax_ = am;
    n_pos_ += 1;
}

int Model::sample(float temperature, float top_p, std::mt19937& rng) {
    if (temperature <= 0.0f) return last_argmax_;
    std::uniform_real_distribution<float> dist(0.0f, 1.0f);
    const float r = dist(rng);
    int32_t tok = -1;
    check(tf_hip_sample(ctx_, temperature, top_p, r, &tok), "sample");
    return tok;
}

void Model::generate(int n, int32_t* out_tokens) {
    if (n <= 0) return;
    if (n > cfg_.max_seq - n_pos_) throw std::runtime_error("decode exceeds max_seq");
    check(tf_hip_generate(ctx_, n, out_tokens), "generate");
    n_pos_ += n;
}

void Model::reset() {
    check(tf_hip_reset(ctx_), "reset");
    n_pos_ = 0;
    last_argmax_ = -1;
}

double Model::decode_bytes(int pos) const { return traffic_.at(pos); }

std::string Model::describe() const {
    std::ostringstream o;
    o << "arch=" << gguf_.arch() << " layers=" << n_layer_ << " dim=" << n_embd_ << " heads=" << n_head_ << "/"
      << n_kv_head_ << " ff=" << n_ff_ << " vocab=" << n_vocab_ << " weights=" << (weight_bytes() / 1e6) << " MB"
      << " stage=" << cfg_.stage << " backend=hip device=" << cfg_.device
      << " kv=" << (cfg_.kv_layout == KVLayout::HeadMajor ? "head" : "seq") << " max_seq=" << cfg_.max_seq;
    return o.str();
}

}  // namespace tfh
