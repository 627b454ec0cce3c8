/*
 * oracle.h - CPU restatement of tinferno's --stage v2 token loop.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the oracle that the HIP backend is
 * compared against. Only tests/, __graft_entry__.smoke() and bench.py's CPU
 * baseline leg load it; the product (libtf_hip.so, libtinferno.so, the CLI)
 * never links, loads or calls it.
 *
 * Each function restates the reference function named in its comment
 * (file:line in the reference's src/), including the operation order of the
 * AVX2 build (-O3 -mavx2 -mfma -mf16c, default FP contraction): every fused
 * multiply-add that g++ emits there is an explicit fmaf() here, everything else
 * is compiled with -ffp-contract=off. The results are meant to be bit-identical
 * to the compiled reference; tests/test_oracle.py checks that.
 */
#ifndef TF_ORACLE_H
#define TF_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (tensor.cpp:18-28) */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_Q4_0 = 2, ORC_Q4_1 = 3, ORC_Q8_0 = 8, ORC_Q6_K = 14 };

/* formats: quant.cpp / tensor.cpp */
float orc_f16_to_f32(uint16_t h);                                   /* quant.cpp:16-45 */
int64_t orc_row_nbytes(int type, int64_t ne0);                      /* tensor.cpp:66-70; -1 if invalid */
int orc_dequant_row(int type, const void* row, int64_t n, float* out); /* quant.cpp:133-145 */
float orc_dot_f32(const float* a, const float* b, int n);           /* quant.cpp:198-214 (simd) */
float orc_dot_row(int type, const float* x, const void* row, int64_t k); /* matmul.cpp:5-20 (v2) */
/* C[M,N] = A[M,K] . W[N,K]^T  (matmul.cpp:22-32, 64-73 with v2: never blocked) */
int orc_matmul(float* c, const float* a, int m, int type, const void* w, int64_t n, int64_t k, int n_threads);

/* layers.cpp */
void orc_rmsnorm(float* out, const float* x, const float* w, int n, float eps); /* :7-12 */
void orc_silu_mul(float* gate, const float* up, int n);                          /* :14-19 */
void orc_softmax(float* x, int n);                                               /* :25-35 */

/* attention.cpp */
void orc_rope_freqs(float* freq, int n_rot, float theta, int llama3, float scale, float low_freq_f,
                    float high_freq_f, float orig_ctx);                          /* :9-29 */
void orc_rope(float* x, int n_heads, int head_dim, int pos, const float* freq); /* :31-46 */
/* one layer's caches; layout 0 = seq-major [pos][kvh][hd], 1 = head-major [kvh][pos][hd] */
void orc_attn_decode(float* out, const float* q, const float* kc, const float* vc, int layout, int n_kv_heads,
                     int max_seq, int n_heads, int head_dim, int n_pos, float* scores); /* :55-80 */
void orc_attn_prefill(float* out, const float* q, const float* k, const float* v, int seq, int n_heads,
                      int n_kv_heads, int head_dim, float* scores);             /* :82-111 */

/* sampler.cpp:8-13: first maximum wins */
int orc_argmax(const float* x, int n);
/* The draws of sample_logits (sampler.cpp:44-45) from std::mt19937(seed): the 32-bit
 * Mersenne Twister (Matsumoto & Nishimura 1998), and libstdc++'s
 * uniform_real_distribution<float>(0, 1) over it (generate_canonical<float, 24>: one
 * draw u, (float)u / 2^32, 1 - 2^-24 when that rounds to 1). n draws in order. */
void orc_uniform_draws(uint32_t seed, int n, float* out);
/* sample_logits (sampler.cpp:15-52) for the uniform draw r: temperature <= 0 is greedy.
 * Optional outputs (may be NULL): the order (descending logits, ties: lower index first;
 * std::sort leaves the order of ties unspecified), the final probabilities in that order
 * (after the nucleus renormalisation) and the nucleus size. */
int orc_sample_logits(const float* logits, int n, float temperature, float top_p, float r, int32_t* sorted_idx,
                      float* probs, int* n_last);

/* model.cpp: Model(path, cfg), prefill, decode, reset */
typedef struct orc_model orc_model;
orc_model* orc_open(const char* path, int max_seq, int kv_layout, int n_threads, char* err, int err_len);
void orc_close(orc_model* m);
int orc_prefill(orc_model* m, const int32_t* tokens, int n, float* logits); /* model.cpp:183-195 */
int orc_decode(orc_model* m, int32_t token, float* logits);                 /* model.cpp:197-208 */
void orc_reset(orc_model* m);                                               /* model.cpp:80-83 */
/* out[0..9] = vocab, embd, ff, layers, heads, kv_heads, head_dim, n_pos, max_seq, kv_layout */
void orc_info(const orc_model* m, int32_t* out);
float orc_rms_eps(const orc_model* m);
/* residual stream after layer l (l < n_layer) or the final-normed vector (l == n_layer), for the
 * last token processed by decode, or the last row of the last prefill */
int orc_tap(const orc_model* m, int layer, float* out);
/* logical K (which=0) or V (which=1) rows [pos0, pos0+n) of one layer as [n][kv_heads][head_dim] */
int orc_read_kv(const orc_model* m, int layer, int which, int pos0, int n, float* out);
const char* orc_last_error(const orc_model* m);

#ifdef __cplusplus
}
#endif
#endif
