#include "synth.hpp"

#include "gguf.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <stdexcept>
#include <thread>

namespace tfh {

// ---------------------------------------------------------------- f16

uint16_t f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);   // NaN
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);  // rounds to +-inf
    if (ax >= 0x38800000u) {                                   // normal half
        const uint32_t m = ax - 0x38000000u;                   // rebias 127 -> 15
        return (uint16_t)(sign | ((m + 0x0FFFu + ((m >> 13) & 1u)) >> 13));
    }
    float v;
    std::memcpy(&v, &ax, 4);
    // subnormal half: v * 2^24 is exact and below 1024; nearbyint rounds half to even
    return (uint16_t)(sign | (uint32_t)std::nearbyint(v * 16777216.0f));
}

float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    const uint32_t m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {  // subnormal: m * 2^-24 is exact in fp32
            float v = (float)m * 5.9604644775390625e-8f;
            std::memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// ---------------------------------------------------------------- quantizers

namespace {

void put_u16(uint8_t* p, uint16_t v) { std::memcpy(p, &v, 2); }

// quant.cpp:147-163 (d = amax/127, q = round(x/d) clamped to +-127)
void quant_q8_0(const float* x, int64_t n, uint8_t* out) {
    for (int64_t b = 0; b < n / 32; ++b, x += 32, out += 34) {
        float amax = 0;
        for (int j = 0; j < 32; ++j) amax = std::max(amax, std::fabs(x[j]));
        const float d = amax / 127.0f;
        const float id = d > 0 ? 1.0f / d : 0.0f;
        put_u16(out, f32_to_f16(d));
        for (int j = 0; j < 32; ++j) {
            int q = (int)std::round(x[j] * id);
            q = std::min(127, std::max(-127, q));
            out[2 + j] = (uint8_t)(int8_t)q;
        }
    }
}

// quant.cpp:165-183 (d = amax/8, nibbles hold q+8 in [0,15], element j low / j+16 high)
void quant_q4_0(const float* x, int64_t n, uint8_t* out) {
    for (int64_t b = 0; b < n / 32; ++b, x += 32, out += 18) {
        float amax = 0;
        for (int j = 0; j < 32; ++j) amax = std::max(amax, std::fabs(x[j]));
        const float d = amax / 8.0f;
        const float id = d > 0 ? 1.0f / d : 0.0f;
        put_u16(out, f32_to_f16(d));
        for (int j = 0; j < 16; ++j) {
            int lo = (int)std::round(x[j] * id);
            int hi = (int)std::round(x[j + 16] * id);
            lo = std::min(7, std::max(-8, lo));
            hi = std::min(7, std::max(-8, hi));
            out[2 + j] = (uint8_t)((lo + 8) | ((hi + 8) << 4));
        }
    }
}

// Q4_1: value = q*d + m with q in [0,15] (the dequant of quant.cpp:87-99).
void quant_q4_1(const float* x, int64_t n, uint8_t* out) {
    for (int64_t b = 0; b < n / 32; ++b, x += 32, out += 20) {
        float lo = x[0], hi = x[0];
        for (int j = 1; j < 32; ++j) {
            lo = std::min(lo, x[j]);
            hi = std::max(hi, x[j]);
        }
        const float d = (hi - lo) / 15.0f;
        const float id = d > 0 ? 1.0f / d : 0.0f;
        put_u16(out, f32_to_f16(d));
        put_u16(out + 2, f32_to_f16(lo));
        for (int j = 0; j < 16; ++j) {
            int a = (int)std::round((x[j] - lo) * id);
            int c = (int)std::round((x[j + 16] - lo) * id);
            a = std::min(15, std::max(0, a));
            c = std::min(15, std::max(0, c));
            out[4 + j] = (uint8_t)(a | (c << 4));
        }
    }
}

// Q6_K: 256-element super-block, 16 sub-blocks of 16 with int8 scales, 6-bit q in
// [-32,31], value = d * sc[e/16] * q. Bit placement is the one quant.cpp:101-127
// decodes: element e = 128h + 32k + l (l < 32) keeps its low nibble in
// ql[64h + l + 32(k&1)] (high nibble when k >= 2) and its top two bits at
// qh[32h + l] bits 2k..2k+1.
void quant_q6_k(const float* x, int64_t n, uint8_t* out) {
    for (int64_t b = 0; b < n / 256; ++b, x += 256, out += 210) {
        float sub_scale[16];
        float max_abs_scale = 0;
        for (int s = 0; s < 16; ++s) {
            float amax = 0, vmax = 0;
            for (int j = 0; j < 16; ++j) {
                const float v = x[16 * s + j];
                if (std::fabs(v) > amax) {
                    amax = std::fabs(v);
                    vmax = v;
                }
            }
            // map the largest-magnitude value to -32 (the wider side of [-32,31])
            sub_scale[s] = amax > 0 ? -vmax / 32.0f : 0.0f;
            max_abs_scale = std::max(max_abs_scale, std::fabs(sub_scale[s]));
        }
        const float d = max_abs_scale / 127.0f;
        const uint16_t d16 = f32_to_f16(d);
        const float dq = f16_to_f32(d16);
        int8_t sc[16];
        for (int s = 0; s < 16; ++s) {
            int v = dq > 0 ? (int)std::round(sub_scale[s] / dq) : 0;
            sc[s] = (int8_t)std::min(127, std::max(-128, v));
        }
        uint8_t q[256];
        for (int e = 0; e < 256; ++e) {
            const float step = dq * (float)sc[e / 16];
            int v = step != 0 ? (int)std::round(x[e] / step) : 0;
            v = std::min(31, std::max(-32, v));
            q[e] = (uint8_t)(v + 32);
        }
        uint8_t* ql = out;
        uint8_t* qh = out + 128;
        std::memset(ql, 0, 128 + 64);
        for (int h = 0; h < 2; ++h)
            for (int k = 0; k < 4; ++k)
                for (int l = 0; l < 32; ++l) {
                    const uint8_t u = q[128 * h + 32 * k + l];
                    uint8_t& lo = ql[64 * h + l + 32 * (k & 1)];
                    lo |= (k < 2) ? (u & 0x0F) : (uint8_t)((u & 0x0F) << 4);
                    qh[32 * h + l] |= (uint8_t)((u >> 4) << (2 * k));
                }
        std::memcpy(out + 192, sc, 16);
        put_u16(out + 208, d16);
    }
}

}  // namespace

void quantize_row(int t, const float* x, int64_t n, uint8_t* out) {
    switch (t) {
        case GGML_F32: std::memcpy(out, x, (size_t)n * 4); break;
        case GGML_F16:
            for (int64_t i = 0; i < n; ++i) put_u16(out + 2 * i, f32_to_f16(x[i]));
            break;
        case GGML_Q8_0: quant_q8_0(x, n, out); break;
        case GGML_Q4_0: quant_q4_0(x, n, out); break;
        case GGML_Q4_1: quant_q4_1(x, n, out); break;
        case GGML_Q6_K: quant_q6_k(x, n, out); break;
        default: throw std::runtime_error("quantize_row: unsupported type");
    }
}

// ---------------------------------------------------------------- random numbers

namespace {

inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline uint64_t stream_key(uint64_t seed, uint64_t stream) {
    return mix64(mix64(seed + 0x9E3779B97F4A7C15ull) ^ (stream * 0xD1B54A32D192ED03ull + 1));
}

// Standard normal from one 64-bit draw: Box-Muller on two 24-bit uniforms.
inline double normal_at(uint64_t key, uint64_t i) {
    const uint64_t r = mix64(key + i * 0x9E3779B97F4A7C15ull);
    const double u1 = ((double)(r >> 40) + 1.0) * (1.0 / 16777216.0);  // (0, 1]
    const double u2 = (double)(r & 0xFFFFFFull) * (1.0 / 16777216.0);  // [0, 1)
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

const uint64_t kPromptStream = 0x50524F4D5054ull;  // "PROMPT"

}  // namespace

std::vector<int32_t> synth_prompt(uint64_t seed, int n, int n_vocab) {
    std::vector<int32_t> ids((size_t)std::max(0, n));
    const uint64_t key = stream_key(seed, kPromptStream);
    for (int i = 0; i < n; ++i) ids[(size_t)i] = (int32_t)(mix64(key + (uint64_t)i) % (uint64_t)n_vocab);
    return ids;
}

// ---------------------------------------------------------------- presets

bool synth_preset(const std::string& name, SynthSpec* s) {
    SynthSpec p;
    p.name = name;
    if (name == "llama1b_q8" || name == "llama1b_mixq4") {
        // Llama-3.2-1B shape: 16 layers, d 2048, 32/8 heads, hd 64, ff 8192, vocab 128256, tied
        p.arch = "llama";
        p.n_vocab = 128256; p.n_embd = 2048; p.n_ff = 8192; p.n_layer = 16; p.n_head = 32; p.n_kv_head = 8;
        p.rope_theta = 500000.0f;
        p.rms_eps = 1e-5f;
        if (name == "llama1b_mixq4") {
            p.type_matrix = GGML_Q4_0;
            p.type_embd = GGML_Q6_K;
            p.overrides = {{0, "ffn_down", GGML_Q4_1}, {15, "ffn_down", GGML_Q4_1}};
        }
    } else if (name == "qwen05b_q8") {
        // Qwen2.5-0.5B shape: 24 layers, d 896, 14/2 heads, hd 64, ff 4864, vocab 151936, QKV bias, tied
        p.arch = "qwen2";
        p.n_vocab = 151936; p.n_embd = 896; p.n_ff = 4864; p.n_layer = 24; p.n_head = 14; p.n_kv_head = 2;
        p.rope_theta = 1000000.0f;
        p.rms_eps = 1e-6f;
        p.bias = true;
    } else if (name == "qwen15b_q8") {
        // Qwen2.5-1.5B shape: 28 layers, d 1536, 12/2 heads, hd 128, ff 8960, vocab 151936, QKV bias, tied
        p.arch = "qwen2";
        p.n_vocab = 151936; p.n_embd = 1536; p.n_ff = 8960; p.n_layer = 28; p.n_head = 12; p.n_kv_head = 2;
        p.rope_theta = 1000000.0f;
        p.rms_eps = 1e-6f;
        p.bias = true;
    } else if (name == "tiny_f32") {
        // The reference CI model's shape (test_correctness.cpp:29-85): all F32, untied, random norms.
        p.n_vocab = 64; p.n_embd = 32; p.n_ff = 64; p.n_layer = 2; p.n_head = 4; p.n_kv_head = 2;
        p.seed = 12345;
        p.tied = false;
        p.norms_random = true;
        p.type_matrix = p.type_embd = p.type_output = GGML_F32;
    } else if (name == "tiny_q8") {
        p.n_vocab = 512; p.n_embd = 128; p.n_ff = 384; p.n_layer = 2; p.n_head = 4; p.n_kv_head = 2;
        p.rope_theta = 500000.0f;
    } else if (name == "tiny_mixq4") {
        p.n_vocab = 512; p.n_embd = 256; p.n_ff = 512; p.n_layer = 3; p.n_head = 4; p.n_kv_head = 2;
        p.rope_theta = 500000.0f;
        p.type_matrix = GGML_Q4_0;
        p.type_embd = GGML_Q6_K;
        p.overrides = {{0, "ffn_down", GGML_Q4_1}, {2, "ffn_down", GGML_Q4_1}};
    } else if (name == "tiny_mixfmt") {
        // a format per matrix: q, k and v in different ones, Q4_1 and F16 gate / up pairs, F32 q
        // and ffn_down, a Q6_K attention output
        p.n_vocab = 512; p.n_embd = 256; p.n_ff = 512; p.n_layer = 2; p.n_head = 4; p.n_kv_head = 2;
        p.rope_theta = 500000.0f;
        p.overrides = {{0, "attn_q", GGML_F16},      {0, "attn_k", GGML_Q4_0},   {0, "attn_v", GGML_Q4_1},
                       {0, "attn_output", GGML_Q6_K}, {0, "ffn_gate", GGML_Q4_1}, {0, "ffn_up", GGML_Q4_1},
                       {0, "ffn_down", GGML_F16},     {1, "attn_q", GGML_F32},    {1, "attn_output", GGML_Q4_1},
                       {1, "ffn_gate", GGML_F16},     {1, "ffn_up", GGML_F16},    {1, "ffn_down", GGML_F32}};
    } else if (name == "tiny_qwen") {
        p.arch = "qwen2";
        p.n_vocab = 640; p.n_embd = 192; p.n_ff = 320; p.n_layer = 2; p.n_head = 6; p.n_kv_head = 1;
        p.rope_theta = 1000000.0f;
        p.rms_eps = 1e-6f;
        p.bias = true;
    } else if (name == "tiny_hd128") {
        // head_dim 128 with 6 query heads per kv head and QKV bias, as the Qwen2.5-1.5B shape
        p.arch = "qwen2";
        p.n_vocab = 1024; p.n_embd = 768; p.n_ff = 1024; p.n_layer = 2; p.n_head = 6; p.n_kv_head = 1;
        p.rope_theta = 1000000.0f;
        p.rms_eps = 1e-6f;
        p.bias = true;
    } else if (name == "small_q8") {
        // mid-size Llama-like model for parity at realistic row lengths (hd 64, GQA 4)
        p.n_vocab = 4096; p.n_embd = 512; p.n_ff = 1536; p.n_layer = 4; p.n_head = 8; p.n_kv_head = 2;
        p.rope_theta = 500000.0f;
    } else {
        return false;
    }
    *s = p;
    return true;
}

std::vector<std::string> synth_preset_names() {
    return {"llama1b_q8", "qwen05b_q8", "llama1b_mixq4", "qwen15b_q8",
            "tiny_f32",   "tiny_q8",    "tiny_mixq4",    "tiny_qwen", "tiny_hd128", "small_q8",
            "tiny_mixfmt"};
}

// ---------------------------------------------------------------- writer

namespace {

struct Planned {
    std::string name;
    int ndim;
    int64_t ne0, ne1;
    int type;
    int kind;  // 0 = normal(w_sigma), 1 = ones, 2 = normal(b_sigma) bias
    uint64_t offset = 0;
    size_t nbytes = 0;
};

struct Blob {
    std::vector<uint8_t> b;
    template <typename T>
    void put(T v) {
        const size_t n = b.size();
        b.resize(n + sizeof(T));
        std::memcpy(b.data() + n, &v, sizeof(T));
    }
    void str(const std::string& s) {
        put<uint64_t>(s.size());
        b.insert(b.end(), s.begin(), s.end());
    }
    void kv_u64(const std::string& k, uint64_t v) { str(k); put<uint32_t>(10); put<uint64_t>(v); }
    void kv_u32(const std::string& k, uint32_t v) { str(k); put<uint32_t>(4); put<uint32_t>(v); }
    void kv_f32(const std::string& k, float v) { str(k); put<uint32_t>(6); put<float>(v); }
    void kv_str(const std::string& k, const std::string& v) { str(k); put<uint32_t>(8); str(v); }
};

int type_for(const SynthSpec& s, int layer, const std::string& suffix) {
    for (const auto& o : s.overrides)
        if (o.layer == layer && o.tensor == suffix) return o.type;
    return s.type_matrix;
}

}  // namespace

uint64_t synth_write(const SynthSpec& s, const std::string& path, int n_threads) {
    if (s.n_head <= 0 || s.n_kv_head <= 0 || s.n_embd % s.n_head != 0 || s.n_head % s.n_kv_head != 0)
        throw std::runtime_error("synth: inconsistent head counts");
    const int64_t hd = s.n_embd / s.n_head;
    const int64_t D = s.n_embd, F = s.n_ff, Hq = s.n_head * hd, Hkv = s.n_kv_head * hd;

    std::vector<Planned> plan;
    plan.push_back({"token_embd.weight", 2, D, s.n_vocab, s.type_embd, 0});
    plan.push_back({"output_norm.weight", 1, D, 1, GGML_F32, s.norms_random ? 0 : 1});
    if (!s.tied) plan.push_back({"output.weight", 2, D, s.n_vocab, s.type_output, 0});
    for (int l = 0; l < s.n_layer; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        plan.push_back({p + "attn_norm.weight", 1, D, 1, GGML_F32, s.norms_random ? 0 : 1});
        plan.push_back({p + "attn_q.weight", 2, D, Hq, type_for(s, l, "attn_q"), 0});
        plan.push_back({p + "attn_k.weight", 2, D, Hkv, type_for(s, l, "attn_k"), 0});
        plan.push_back({p + "attn_v.weight", 2, D, Hkv, type_for(s, l, "attn_v"), 0});
        if (s.bias) {
            plan.push_back({p + "attn_q.bias", 1, Hq, 1, GGML_F32, 2});
            plan.push_back({p + "attn_k.bias", 1, Hkv, 1, GGML_F32, 2});
            plan.push_back({p + "attn_v.bias", 1, Hkv, 1, GGML_F32, 2});
        }
        plan.push_back({p + "attn_output.weight", 2, Hq, D, type_for(s, l, "attn_output"), 0});
        plan.push_back({p + "ffn_norm.weight", 1, D, 1, GGML_F32, s.norms_random ? 0 : 1});
        plan.push_back({p + "ffn_gate.weight", 2, D, F, type_for(s, l, "ffn_gate"), 0});
        plan.push_back({p + "ffn_up.weight", 2, D, F, type_for(s, l, "ffn_up"), 0});
        plan.push_back({p + "ffn_down.weight", 2, F, D, type_for(s, l, "ffn_down"), 0});
    }
    const uint64_t align = 32;
    uint64_t acc = 0, weight_bytes = 0;
    for (auto& t : plan) {
        t.nbytes = (size_t)t.ne1 * ggml_row_nbytes(t.type, t.ne0);
        t.offset = acc;
        acc = (acc + t.nbytes + align - 1) / align * align;
        weight_bytes += t.nbytes;
    }

    Blob h;
    const std::string a = s.arch;
    h.put<uint32_t>(0x46554747u);
    h.put<uint32_t>(3);
    h.put<uint64_t>(plan.size());
    const uint64_t n_kv = 22 + (s.write_vocab ? 1 : 0);
    h.put<uint64_t>(n_kv);
    h.kv_str("general.architecture", a);
    h.kv_str("general.name", "synthetic-" + s.name);
    h.kv_u32("general.alignment", (uint32_t)align);
    h.kv_u64(a + ".vocab_size", (uint64_t)s.n_vocab);
    h.kv_u64(a + ".context_length", 131072);
    h.kv_u64(a + ".embedding_length", (uint64_t)s.n_embd);
    h.kv_u64(a + ".feed_forward_length", (uint64_t)s.n_ff);
    h.kv_u64(a + ".block_count", (uint64_t)s.n_layer);
    h.kv_u64(a + ".attention.head_count", (uint64_t)s.n_head);
    h.kv_u64(a + ".attention.head_count_kv", (uint64_t)s.n_kv_head);
    h.kv_u64(a + ".rope.dimension_count", (uint64_t)hd);
    h.kv_f32(a + ".rope.freq_base", s.rope_theta);
    h.kv_f32(a + ".attention.layer_norm_rms_epsilon", s.rms_eps);
    h.kv_str("tokenizer.ggml.model", "gpt2");
    h.kv_u64("tokenizer.ggml.bos_token_id", 1);
    h.kv_u64("tokenizer.ggml.eos_token_id", 2);
    h.kv_str("synthetic.preset", s.name);
    h.kv_u64("synthetic.seed", s.seed);
    h.kv_f32("synthetic.weight_sigma", s.w_sigma);
    h.kv_f32("synthetic.bias_sigma", s.b_sigma);
    h.kv_str("synthetic.rng", "splitmix64 counter + Box-Muller (24-bit uniforms), element e of tensor t");
    h.kv_str("synthetic.norms", s.norms_random ? "normal" : "ones");
    if (s.write_vocab) {
        h.str("tokenizer.ggml.tokens");
        h.put<uint32_t>(9);
        h.put<uint32_t>(8);
        h.put<uint64_t>((uint64_t)s.n_vocab);
        for (int i = 0; i < s.n_vocab; ++i) h.str("tok" + std::to_string(i));
    }
    for (const auto& t : plan) {
        h.str(t.name);
        h.put<uint32_t>((uint32_t)t.ndim);
        h.put<uint64_t>((uint64_t)t.ne0);
        if (t.ndim == 2) h.put<uint64_t>((uint64_t)t.ne1);
        h.put<uint32_t>((uint32_t)t.type);
        h.put<uint64_t>(t.offset);
    }
    const uint64_t data_off = (h.b.size() + align - 1) / align * align;
    const uint64_t total = data_off + acc;

    const int fd = ::open(path.c_str(), O_RDWR | O_CREAT | O_TRUNC, 0644);
    if (fd < 0) throw std::runtime_error("cannot write " + path);
    if (ftruncate(fd, (off_t)total) != 0) {
        ::close(fd);
        throw std::runtime_error("ftruncate failed: " + path);
    }
    void* m = mmap(nullptr, total, PROT_READ | PROT_WRITE, MAP_SHARED, fd, 0);
    if (m == MAP_FAILED) {
        ::close(fd);
        throw std::runtime_error("mmap failed: " + path);
    }
    uint8_t* base = (uint8_t*)m;
    std::memcpy(base, h.b.data(), h.b.size());

    // Work items: (tensor, row chunk). Each element's value depends only on (seed, t, e).
    struct Item {
        size_t t;
        int64_t r0, r1;
    };
    std::vector<Item> items;
    for (size_t t = 0; t < plan.size(); ++t) {
        const int64_t rows = plan[t].ne1;
        const int64_t chunk = std::max<int64_t>(1, (1 << 20) / std::max<int64_t>(1, plan[t].ne0));
        for (int64_t r = 0; r < rows; r += chunk) items.push_back({t, r, std::min(rows, r + chunk)});
    }
    int nt = n_threads > 0 ? n_threads : (int)std::thread::hardware_concurrency();
    nt = std::max(1, std::min(nt, 16));
    std::atomic<size_t> next{0};
    auto worker = [&]() {
        std::vector<float> row;
        for (;;) {
            const size_t i = next.fetch_add(1);
            if (i >= items.size()) return;
            const Item& it = items[i];
            const Planned& t = plan[it.t];
            const uint64_t key = stream_key(s.seed, it.t);
            const size_t rb = ggml_row_nbytes(t.type, t.ne0);
            row.resize((size_t)t.ne0);
            for (int64_t r = it.r0; r < it.r1; ++r) {
                for (int64_t c = 0; c < t.ne0; ++c) {
                    if (t.kind == 1) {
                        row[(size_t)c] = 1.0f;
                    } else {
                        const double sig = t.kind == 2 ? s.b_sigma : s.w_sigma;
                        row[(size_t)c] = (float)(sig * normal_at(key, (uint64_t)(r * t.ne0 + c)));
                    }
                }
                quantize_row(t.type, row.data(), t.ne0, base + data_off + t.offset + (size_t)r * rb);
            }
        }
    };
    std::vector<std::thread> pool;
    for (int i = 1; i < nt; ++i) pool.emplace_back(worker);
    worker();
    for (auto& th : pool) th.join();
    munmap(m, total);
    ::close(fd);
    return weight_bytes;
}

}  // namespace tfh
