// Model API of the reference (model.hpp:24-90, common.hpp:103-116 and 289-322) over the
// MI355X backend: the same constructor, prefill/decode/reset and accessors, with the
// token loop running in libtf_hip (include/tf_hip.h). Errors surface as
// std::runtime_error, as in the reference.
#pragma once

#include <cstdint>
#include <memory>
#include <random>
#include <string>
#include <vector>

#include "gguf.hpp"
#include "tf_hip.h"

namespace tfh {

enum class KVLayout { SeqMajor, HeadMajor };

// RunConfig of common.hpp:103-116. The HIP backend reads max_seq, kv_layout and device;
// n_threads/use_simd/use_blocking keep their reference meaning for the CPU stages and
// only label a run here.
struct RunConfig {
    int n_threads = 1;
    bool use_simd = false;
    bool use_blocking = false;
    KVLayout kv_layout = KVLayout::SeqMajor;
    int n_predict = 64;
    float temperature = 0.0f;
    float top_p = 0.9f;
    int seed = 42;
    int max_seq = 4096;
    bool pin_threads = false;
    bool profile = false;
    std::string stage = "v2";
    int device = 0;
};

// stage_preset of common.hpp:289-322 (v0..v5; throws on an unknown stage).
RunConfig stage_preset(const std::string& stage, int hw_threads);

// rope_freqs of attention.cpp:9-29 and the per-position angles of rope_one
// (attention.cpp:31-41): cos/sin of (float)pos * freq[i], [n_pos][n_rot/2].
struct RopeParams {
    bool llama3 = false;
    float theta = 10000.0f;
    int n_rot = 0;
    float scale = 1.0f, low_freq_f = 1.0f, high_freq_f = 4.0f, orig_ctx = 8192.0f;
};
std::vector<float> rope_freqs(const RopeParams& rp);
void rope_tables(const std::vector<float>& freq, int n_pos, std::vector<float>& cos_tab, std::vector<float>& sin_tab);

// Hyperparameters exactly as model.cpp:9-41 derives them from the GGUF metadata.
struct HParams {
    int n_vocab = 0, n_embd = 0, n_ff = 0, n_layer = 0, n_head = 0, n_kv_head = 0, head_dim = 0;
    int bos = 1, eos = 2;
    float rms_eps = 1e-5f;
    RopeParams rope;
};
HParams read_hparams(const GgufFile& g);

// Algorithmic bytes of one decode step (the roofline's numerator): every tensor the step
// reads once -- the layer matrices, norms and biases, the lm_head (token_embd when tied)
// -- plus one embedding row, plus K and V rows of every attended position and the new
// row written. decode_bytes(pos) = tensor_bytes + embd_row_bytes + kv_bytes_per_pos * (pos + 2).
struct DecodeTraffic {
    size_t tensor_bytes = 0;
    size_t embd_row_bytes = 0;
    double kv_bytes_per_pos = 0;  // n_layer * n_kv_head * head_dim * 4 * 2 (fp32 K and V)
    double at(int pos) const { return (double)tensor_bytes + (double)embd_row_bytes + kv_bytes_per_pos * (pos + 2); }
};
DecodeTraffic decode_traffic(const GgufFile& g, const HParams& hp);

class Model {
public:
    Model(const std::string& path, const RunConfig& cfg);
    ~Model();
    Model(const Model&) = delete;
    Model& operator=(const Model&) = delete;

    // Model::prefill / decode / reset (model.cpp:80-83, 183-208). logits may be null.
    void prefill(const int* tokens, int n, float* logits);
    void decode(int token, float* logits);
    void reset();

    // Greedy argmax of the logits of the last prefill/decode (sample_greedy on them).
    int last_argmax() const { return last_argmax_; }
    // The greedy loop on the device: n tokens, as n x (sample_greedy + decode).
    void generate(int n, int32_t* out_tokens);
    // sample_logits (sampler.cpp:15-52) of the last step's logits on the GPU: temperature
    // <= 0 is the greedy argmax and draws nothing from rng; otherwise one
    // uniform_real_distribution<float>(0, 1) draw, as the reference makes.
    int sample(float temperature, float top_p, std::mt19937& rng);

    int n_vocab() const { return n_vocab_; }
    int n_embd() const { return n_embd_; }
    int n_ff() const { return n_ff_; }
    int n_layer() const { return n_layer_; }
    int n_head() const { return n_head_; }
    int n_kv_head() const { return n_kv_head_; }
    int head_dim() const { return head_dim_; }
    int n_pos() const { return n_pos_; }
    int bos() const { return bos_; }
    int eos() const { return eos_; }
    float rms_eps() const { return rms_eps_; }
    size_t weight_bytes() const { return gguf_.weight_bytes(); }
    // Bytes one decode step reads at position pos (all weights once, one embedding row,
    // the KV cache over pos+1 positions) -- the algorithmic traffic of the roofline.
    double decode_bytes(int pos) const;
    const GgufFile& gguf() const { return gguf_; }
    const RunConfig& cfg() const { return cfg_; }
    tf_hip_ctx* ctx() { return ctx_; }
    std::string describe() const;

private:
    void check(int rc, const char* what) const;
    GgufFile gguf_;
    RunConfig cfg_;
    tf_hip_ctx* ctx_ = nullptr;
    int n_vocab_ = 0, n_embd_ = 0, n_ff_ = 0, n_layer_ = 0, n_head_ = 0, n_kv_head_ = 0, head_dim_ = 0;
    int bos_ = 1, eos_ = 2;
    float rms_eps_ = 1e-5f;
    int n_pos_ = 0;
    int last_argmax_ = -1;
    DecodeTraffic traffic_;
};

}  // namespace tfh
