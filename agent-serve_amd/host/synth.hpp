// Seeded synthetic GGUF writer for the Llama/Qwen-shaped workloads of the token loop.
//
// The reference ships a minimal F32-only writer (gguf.cpp:237-300) and builds its
// CI model with std::normal_distribution (test_correctness.cpp:29-85), whose output
// depends on the standard library. This writer is counter-based instead: element e
// of tensor t is a Box-Muller normal of splitmix64(seed, t, e), so files are
// identical on every machine and can be generated in parallel. Quantizers follow the
// reference's for Q8_0 and Q4_0 (quant.cpp:147-183); Q4_1 and Q6_K have none in
// the reference and are written so that the reference dequantizers
// (quant.cpp:87-127) recover them.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace tfh {

struct SynthSpec {
    std::string name = "custom";
    std::string arch = "llama";  // "llama" | "qwen2"
    int n_vocab = 0, n_embd = 0, n_ff = 0, n_layer = 0, n_head = 0, n_kv_head = 0;
    float rope_theta = 10000.0f;
    float rms_eps = 1e-5f;
    uint64_t seed = 42;
    float w_sigma = 0.02f;
    float b_sigma = 0.01f;
    bool bias = false;          // attn_{q,k,v}.bias as F32 (model.cpp:85-89 reads them as raw F32)
    bool tied = true;           // no output.weight: token_embd doubles as lm_head (model.cpp:43-47)
    bool norms_random = false;  // norms N(0, w_sigma) instead of 1.0 (the reference CI model's choice)
    bool write_vocab = true;    // tokenizer.ggml.tokens array
    int type_matrix = 8;        // ggml type of the 7 per-layer matrices
    int type_embd = 8;          // token_embd
    int type_output = 8;        // output.weight when untied
    // (layer, tensor suffix, ggml type) overrides, e.g. {0, "ffn_down", Q4_1}
    struct Override {
        int layer;
        std::string tensor;
        int type;
    };
    std::vector<Override> overrides;
};

// Named presets: llama1b_q8, qwen05b_q8, llama1b_mixq4, qwen15b_q8 (the five
// workloads use these four weight files) plus small test models tiny_f32,
// tiny_q8, tiny_mixq4, tiny_qwen, small_q8.
bool synth_preset(const std::string& name, SynthSpec* out);
std::vector<std::string> synth_preset_names();

// Writes the GGUF; returns its weight bytes. Throws std::runtime_error on I/O errors.
uint64_t synth_write(const SynthSpec& spec, const std::string& path, int n_threads = 0);

// n prompt ids uniform on [0, n_vocab) drawn from the seed (stream independent of the weights).
std::vector<int32_t> synth_prompt(uint64_t seed, int n, int n_vocab);

// IEEE half <-> single, round-to-nearest-even (the F16C behaviour the reference's
// AVX2 build uses, quant.cpp:16-18 and 47-49).
uint16_t f32_to_f16(float f);
float f16_to_f32(uint16_t h);

// Block quantizers (one row of n elements).
void quantize_row(int ggml_type, const float* x, int64_t n, uint8_t* out);

}  // namespace tfh
