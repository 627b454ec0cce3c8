/*
 * tf_hip.h - C ABI of the MI355X (gfx950) backend for tinferno's token loop.
 *
 * The reference runs Model::decode / Model::prefill on CPU threads (model.cpp:183-208)
 * through free functions over raw fp32 pointers: matmul (matmul.hpp:9), apply_rope
 * (attention.hpp:23), attn_decode (attention.hpp:27), rmsnorm/silu_mul/softmax
 * (layers.hpp:7-10), sample_greedy (sampler.hpp:8) and KVCache (kvcache.hpp:7-30).
 * The reference has no FFI of its own; these entry points are what its Model would
 * bind to run the same loop on the GPU. Plain C types only: no exceptions cross
 * this boundary, every call returns a status (0 = ok, negative = error) and the
 * message of the last failure on a context is tf_hip_last_error().
 *
 * Threading: one context per host thread; calls on one context are serialised by
 * the caller, as the reference's Model is (model.hpp:24-90). Host buffers are
 * read/written synchronously: outputs are ready when a call returns.
 */
#ifndef TF_HIP_H
#define TF_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TF_HIP_OK 0
#define TF_HIP_EINVAL -1   /* bad argument, shape or state (std::runtime_error in the reference) */
#define TF_HIP_ERANGE -2   /* max_seq exceeded or token out of range (model.cpp:185, 198) */
#define TF_HIP_ENOMEM -3   /* device allocation failed */
#define TF_HIP_EDEVICE -4  /* HIP runtime error */
#define TF_HIP_ESTATE -5   /* call not allowed in this state (tensors not uploaded, first no-alloc call under capture) */
#define TF_HIP_ESCRATCH -6 /* request larger than a static scratch (tf_hip_attn_decode_noalloc) */

/* ggml tensor types accepted by the token loop (tensor.cpp:18-28) */
#define TF_HIP_TYPE_F32 0
#define TF_HIP_TYPE_F16 1
#define TF_HIP_TYPE_Q4_0 2
#define TF_HIP_TYPE_Q4_1 3
#define TF_HIP_TYPE_Q8_0 8
#define TF_HIP_TYPE_Q6_K 14

/* KV cache layouts (kvcache.cpp:21-29) */
#define TF_HIP_KV_SEQ_MAJOR 0  /* [layer][pos][kv_head][head_dim] */
#define TF_HIP_KV_HEAD_MAJOR 1 /* [layer][kv_head][pos][head_dim] */

/* Model hyperparameters as Model::Model derives them (model.cpp:9-41). */
typedef struct tf_hip_hparams {
    int32_t n_vocab;
    int32_t n_embd;
    int32_t n_ff;
    int32_t n_layer;
    int32_t n_head;
    int32_t n_kv_head;
    int32_t head_dim; /* n_embd / n_head (model.cpp:22-24) */
    int32_t max_seq;  /* RunConfig::max_seq (common.hpp:112) */
    int32_t kv_layout;
    float rms_eps;
} tf_hip_hparams;

/* Tensor slots (the names Model binds, model.cpp:43-65). */
#define TF_HIP_SLOT_TOKEN_EMBD 0  /* token_embd.weight [n_vocab x n_embd] */
#define TF_HIP_SLOT_OUTPUT_NORM 1 /* output_norm.weight F32 [n_embd] */
#define TF_HIP_SLOT_OUTPUT 2      /* output.weight; absent = tied to token_embd (model.cpp:45-46) */
#define TF_HIP_LAYER_ATTN_NORM 0
#define TF_HIP_LAYER_Q 1
#define TF_HIP_LAYER_K 2
#define TF_HIP_LAYER_V 3
#define TF_HIP_LAYER_O 4
#define TF_HIP_LAYER_BQ 5 /* optional F32 biases (model.cpp:58-60, 85-89) */
#define TF_HIP_LAYER_BK 6
#define TF_HIP_LAYER_BV 7
#define TF_HIP_LAYER_FFN_NORM 8
#define TF_HIP_LAYER_GATE 9
#define TF_HIP_LAYER_UP 10
#define TF_HIP_LAYER_DOWN 11
#define TF_HIP_LAYER_COUNT 12
#define TF_HIP_SLOT_LAYER(layer, kind) (16 + (layer) * TF_HIP_LAYER_COUNT + (kind))

typedef struct tf_hip_ctx tf_hip_ctx;

/* Context: device memory for weights, the fp32 KV cache ([n_layer][n_kv_head*max_seq*head_dim]
 * for K and for V, as KVCache::init, kvcache.cpp:5-14), activations and the decode graph.
 * Replaces Model::Model's buffer set-up (model.cpp:67-77). */
int tf_hip_create(int device, const tf_hip_hparams* hp, tf_hip_ctx** out);
int tf_hip_destroy(tf_hip_ctx* ctx);
const char* tf_hip_last_error(const tf_hip_ctx* ctx);

/* Copies one GGUF tensor (raw GGUF row bytes, ne0 = row length, ne1 = rows) to HBM and
 * converts it to the backend's layout. Replaces the mmap binding of model.cpp:43-65. */
int tf_hip_upload_tensor(tf_hip_ctx* ctx, int slot, int ggml_type, int64_t ne0, int64_t ne1, const void* host,
                         size_t nbytes);

/* RoPE angle tables: cos/sin of (float)pos * freq[i] for pos < n_pos, i < half_dim, computed
 * by the host exactly as rope_one does (attention.cpp:31-41) so device and host use
 * identical angles. Row-major [n_pos][half_dim]; n_pos must be >= max_seq. */
int tf_hip_set_rope_table(tf_hip_ctx* ctx, const float* cos_tab, const float* sin_tab, int32_t n_pos,
                          int32_t half_dim);

/* Model::prefill (model.cpp:183-195): consumes tokens[0..n) at positions n_pos.. and writes
 * the last token's logits (n_vocab floats) and/or its greedy argmax. Either output may be
 * NULL. Attention covers only this call's tokens, as attn_prefill does (attention.cpp:82-111). */
int tf_hip_prefill(tf_hip_ctx* ctx, const int32_t* tokens, int32_t n, float* logits, int32_t* argmax);

/* Model::decode (model.cpp:197-208): one token at n_pos, logits and/or argmax (either may be NULL). */
int tf_hip_decode(tf_hip_ctx* ctx, int32_t token, float* logits, int32_t* argmax);

/* The greedy loop of bench_e2e.cpp:49-54 / main.cpp:112-122 run on the device: n times,
 * tok = argmax of the current logits (sample_greedy, sampler.cpp:8-13), out_tokens[i] = tok,
 * decode(tok). Requires a prior prefill or decode. No host round trip between steps. */
int tf_hip_generate(tf_hip_ctx* ctx, int32_t n, int32_t* out_tokens);

/* Decode path of prefill / decode / generate. TF_HIP_PATH_STEP (the default): one
 * persistent cooperative kernel per call runs every token of the call, for models whose
 * layer matrices share one format the kernel is compiled for (Q8_0, F32, or Q4_0 with
 * Q4_1 wo / ffn_down allowed; others use the graph path; tokens attending more than
 * split_from positions, 64 by default, split each layer's attention over workgroups,
 * shorter spans run it on one workgroup per kv head; see tf_hip_set_split_from).
 * TF_HIP_PATH_GRAPH: one captured graph of
 * per-layer kernels replayed per token. Both compute the same function; neither has a
 * counterpart in the reference (a backend choice below Model::decode, model.cpp:197-208).
 * tf_hip_get_decode_path returns the path the next call will take (needs every tensor
 * uploaded). The environment variable TF_HIP_DECODE_PATH (step or graph), read by
 * tf_hip_create, sets the initial path for callers that never call the setter. The step
 * path launches cooperatively; when the GPU refuses the cooperative launch (another
 * process holds that resource, or the grid does not fit), the context switches itself to
 * the graph path for the rest of its life and tf_hip_get_decode_path reports that. */
#define TF_HIP_PATH_GRAPH 0
#define TF_HIP_PATH_STEP 1
int tf_hip_set_decode_path(tf_hip_ctx* ctx, int32_t path);
int tf_hip_get_decode_path(tf_hip_ctx* ctx);

/* Tuning knob of the step kernel's split attention (no counterpart in the reference):
 * spans of more than `span` attended positions split over every workgroup, shorter split
 * ones over the trailing workgroups only. span < 0 restores the
 * model-derived default. Results are the same function either way; used by the tests to
 * place the switch inside a short decode. */
int tf_hip_set_split_all_from(tf_hip_ctx* ctx, int32_t span);

/* Tuning knob of the step kernel's attention (no counterpart in the reference): tokens
 * attending at most `span` positions run attention on one workgroup per kv head, longer
 * spans split it over workgroups. 0 <= span <= 512 (one workgroup per kv head attends at
 * most 512 positions); span < 0 restores the default, 64. Out-of-range spans are rejected
 * with TF_HIP_EINVAL. The environment variable TF_HIP_SPLIT_FROM, read once by
 * tf_hip_create, sets the initial value when it is a whole number in that range. Results
 * are the same function either way. */
int tf_hip_set_split_from(tf_hip_ctx* ctx, int32_t span);

/* The step kernel's attention configuration for this model (no counterpart in the
 * reference): out[0] workgroups of a launch, out[1] splits per kv head of the trailing
 * layout, out[2] splits per kv head when every workgroup splits (0: that layout is not
 * available), out[3] split_from, out[4] the span past which every workgroup splits.
 * n >= 5. Needs every tensor uploaded; TF_HIP_ESTATE when the step kernel does not run
 * this model. */
int tf_hip_get_step_config(tf_hip_ctx* ctx, int32_t* out, int32_t n);

/* Test hook (no counterpart in the reference): sets the step kernel's exchange epoch
 * counter, so that a test can run a launch across the counter's wrap at 2^32 (the kernel
 * then clears its exchange words and starts the count again). */
int tf_hip_set_exchange_epoch(tf_hip_ctx* ctx, uint32_t epoch);

/* The hyperparameters the context was created with (Model's accessors, model.hpp; the
 * device KV cache's layout is out->kv_layout). With the environment variable TF_HIP_LOG
 * set (and not "0"), tf_hip_create also prints them as one line on stderr. */
int tf_hip_get_hparams(const tf_hip_ctx* ctx, tf_hip_hparams* out);

/* Test hook (no counterpart in the reference): the next n launches of the step kernel on
 * this context report the refusal a GPU gives when another process holds its
 * cooperative-launch resource, so a test can check the switch to the graph path. */
int tf_hip_test_refuse_cooperative(tf_hip_ctx* ctx, int32_t n);

/* Prefill path (no counterpart in the reference, whose layer_prefill is the one
 * path, model.cpp:144-195): TF_HIP_PREFILL_MFMA runs a prompt of two or more tokens
 * through the matrix-core GEMMs and the causal chunk attention when every layer
 * matrix is Q8_0, Q4_0, Q4_1, F16, F32 or Q6_K with row lengths divisible by 64 (256 for
 * Q6_K; at most 16384) and output lengths by 16, ffn_gate and ffn_up share a format, the
 * head size is 32, 64 or 128 and a kv head has at most 8 query heads (the default);
 * otherwise, and under TF_HIP_PREFILL_TOKENS, prompt tokens run one at a time through the
 * decode path with attention limited to the prompt. get returns the path a prompt would
 * take (or < 0 on error). */
#define TF_HIP_PREFILL_TOKENS 0
#define TF_HIP_PREFILL_MFMA 1
int tf_hip_set_prefill_path(tf_hip_ctx* ctx, int32_t path);
int tf_hip_get_prefill_path(tf_hip_ctx* ctx);

/* Model::reset (model.cpp:80-83): n_pos = 0 and the KV cache cleared. */
int tf_hip_reset(tf_hip_ctx* ctx);
int tf_hip_get_pos(const tf_hip_ctx* ctx);

/* Parity taps for the last token processed: the residual stream after layer l (l < n_layer),
 * or the output_norm-ed vector fed to the lm_head (l == n_layer); n_embd floats. */
int tf_hip_get_layer_act(tf_hip_ctx* ctx, int32_t layer, float* out);

/* KV rows [pos0, pos0+n) of one layer in logical order [n][n_kv_head][head_dim], K (which = 0)
 * or V (which = 1), whatever the layout (KVCache::k_at / v_at, kvcache.cpp:38-43). */
int tf_hip_read_kv(tf_hip_ctx* ctx, int32_t layer, int32_t which, int32_t pos0, int32_t n, float* out);

/* Timing of the last tf_hip_generate or tf_hip_prefill call, from HIP events on the
 * context's stream: total device milliseconds of the call's kernels, and of the dominant
 * kernel summed over the call together with its launch count; kernel_name names the path
 * ("k_step", "decode_graph", "prefill_mfma"). */
int tf_hip_last_timing(const tf_hip_ctx* ctx, float* total_ms, float* kernel_ms, int32_t* kernel_launches,
                       char* kernel_name, int32_t name_len);

/* The loop of tf_hip_generate with each kernel launched on its own (no graph) and bracketed
 * by HIP events on the context stream. Per kernel class k < TF_HIP_KERNEL_CLASSES it
 * reports the summed device milliseconds, the launch count and the algorithmic bytes (the
 * weights, norm weights and biases each kernel reads; attention the K and V rows it reads
 * and the new row it writes), so that over a step they add up to the decode byte formula
 * (every tensor once + one embedding row + K/V rows). Classes: 0 embedding, 1 QKV GEMV, 2 attention,
 * 3 attn_output GEMV, 4 gate/up GEMV, 5 down GEMV, 6 lm_head GEMV (tf_hip_kernel_class_name). */
#define TF_HIP_KERNEL_CLASSES 7
int tf_hip_profile_generate(tf_hip_ctx* ctx, int32_t n, int32_t* out_tokens, float* ms_by_class,
                            int32_t* launches_by_class, double* bytes_by_class);
const char* tf_hip_kernel_class_name(int32_t k);

/* ---------------------------------------------------------------- op-level entry points
 * Single calls of one backend kernel on host buffers (copied in and out), for the
 * per-op parity tests. They run on `device` with temporary allocations. */

/* dequant_row over rows [row0, row0+nrows) of a GGUF tensor (quant.cpp:133-145): out is
 * [nrows][ne0] fp32. Bit-exact with the reference. */
int tf_hip_dequant_rows(int device, int ggml_type, const void* w, int64_t ne0, int64_t ne1, int64_t row0,
                        int64_t nrows, float* out);

/* matmul (matmul.cpp:64-73): y[m][n] = sum_k x[m][k] * W[n][k] for m < n_rows_x.
 * One row runs the decode GEMV. Two or more rows of a Q8_0, Q4_0, Q4_1, F16, F32 or Q6_K
 * matrix with ne0 % 64 == 0 (Q6_K: % 256), ne0 <= 16384 and ne1 % 16 == 0 run the prefill
 * GEMM on the matrix cores; other shapes run the GEMV once per row. */
int tf_hip_matmul(int device, int ggml_type, const void* w, int64_t ne0, int64_t ne1, const float* x,
                  int32_t n_rows_x, float* y);

/* rmsnorm (layers.cpp:7-12) of n_rows rows of length n. */
int tf_hip_rmsnorm(int device, const float* x, const float* w, int32_t n, int32_t n_rows, float eps, float* out);

/* apply_rope_many (attention.cpp:48-53; apply_rope, attention.cpp:43-46, is seq = 1):
 * rotates x [seq][n_heads][head_dim] in place, row i at position pos0 + i, pairs
 * (x[j], x[j + head_dim/2]) as rope_one (attention.cpp:31-41) with its two contracted
 * products. The angles come from cos_tab / sin_tab [n_pos_tab][head_dim/2], the tables
 * tf_hip_set_rope_table takes (cos/sin((float)pos * freq) on the host), so the result is
 * bit-identical to the reference's. TF_HIP_EINVAL for an odd head_dim or rows past the
 * tables. */
int tf_hip_rope(int device, float* x, int32_t seq, int32_t n_heads, int32_t head_dim, int32_t pos0,
                const float* cos_tab, const float* sin_tab, int32_t n_pos_tab);

/* attn_decode (attention.cpp:55-80) for one layer: q [n_heads][hd] (already rotated),
 * k_rows/v_rows [n_pos][n_kv][hd] logical rows stored into a cache of the given layout and
 * max_seq before the kernel runs; out [n_heads][hd]. */
int tf_hip_attn_decode(int device, const float* q, const float* k_rows, const float* v_rows, int32_t n_heads,
                       int32_t n_kv, int32_t hd, int32_t n_pos, int32_t max_seq, int32_t layout, float* out);

/* attn_decode over a device-resident cache with no allocation at all. No counterpart in
 * the reference: it is for callers that cannot allocate device memory -- code under HIP
 * graph capture, serving loops that forbid hipMalloc. The same function and kernels as
 * tf_hip_attn_decode on the same rows, but every pointer is device memory: q and out
 * [n_heads][hd] (q already rotated), k_cache / v_cache a cache of the given layout and
 * max_seq whose positions [0, n_pos) are filled. The work is enqueued on `stream` (a
 * hipStream_t; NULL for the null stream) and not waited for; nothing is allocated,
 * freed or synchronised. Caches longer than 512 positions split the positions over
 * S = min(512, ceil(max_seq / 32)) workgroups per kv head, whose partials live in the
 * library's static device scratch of TF_HIP_ATTN_SCRATCH_BYTES per GPU (held until the
 * process ends): n_heads * S * (hd + 2) * 4 bytes must fit, else TF_HIP_ESCRATCH before
 * any launch. Every call on a GPU shares that GPU's scratch, so calls that overlap on
 * one GPU (other streams, other host threads) race; each call rewrites every partial it
 * reads, so nothing needs clearing between calls. The first call on each device looks up
 * the scratch's address and must be made outside graph capture (a warm-up call); made on a
 * capturing stream it returns TF_HIP_ESTATE and enqueues nothing. Later calls may be
 * captured: the graph then replays the same kernels on the same scratch. */
#define TF_HIP_ATTN_SCRATCH_BYTES (4u << 20)
int tf_hip_attn_decode_noalloc(int device, const float* q, const float* k_cache, const float* v_cache,
                               int32_t n_heads, int32_t n_kv, int32_t hd, int32_t n_pos, int32_t max_seq,
                               int32_t layout, float* out, void* stream);

/* attn_prefill (attention.cpp:82-111, attention.hpp:29-30): causal GQA attention of seq
 * positions over their own rows. q [seq][n_heads][hd], k and v [seq][n_kv][hd] (already
 * rotated), out [seq][n_heads][hd]; hd 32, 64 or 128, n_heads / n_kv at most 8. */
int tf_hip_attn_prefill(int device, const float* q, const float* k, const float* v, int32_t seq, int32_t n_heads,
                        int32_t n_kv, int32_t hd, float* out);

/* sample_logits (sampler.cpp:15-52) over the logits of the context's last step (its last
 * tf_hip_prefill, tf_hip_decode or tf_hip_generate), for the uniform draw r in [0, 1) that the
 * reference takes from its std::mt19937 (uniform_real_distribution<float>(0, 1),
 * sampler.cpp:44-45; the caller keeps the generator, main.cpp:109). temperature <= 0 is
 * sample_greedy and leaves r unused, as the reference draws nothing then. The logits never
 * leave the GPU; the reference's arithmetic (its libm's expf, the sums in sorted order) picks
 * the reference's token for the same draw. Logits that compare equal are taken in ascending
 * index order (std::sort leaves their order unspecified). TF_HIP_ESTATE before any step. */
int tf_hip_sample(tf_hip_ctx* ctx, float temperature, float top_p, float r, int32_t* token);

/* sample_logits (sampler.cpp:15-52) of n host logits for the draw r, as tf_hip_sample.
 * sorted_idx / probs (n each, may be NULL) receive the descending order and the final
 * probabilities in that order (after the nucleus renormalisation; entries past the nucleus
 * hold p_i / sum). */
int tf_hip_sample_logits(int device, const float* logits, int32_t n, float temperature, float top_p, float r,
                         int32_t* token, int32_t* sorted_idx, float* probs);

/* sample_greedy (sampler.cpp:8-13): index of the first maximum. */
int tf_hip_argmax(int device, const float* x, int32_t n, int32_t* out);

/* Read-only HBM stream (the GPU analogue of bench/stream.c:128-141): sums nbytes of device
 * memory `iters` times; reports the best and median GB/s over the iterations. The buffer
 * holds 32-bit word i = i * 0x9E3779B1 (mod 2^32), summed as integers, so *checksum (may be
 * NULL) is 0x9E3779B1 * n (n - 1) / 2 mod 2^32 for n = nbytes / 16 * 4 words exactly when
 * every word was read. */
int tf_hip_read_stream(int device, size_t nbytes, int32_t iters, double* best_gbs, double* median_gbs,
                       uint32_t* checksum);

/* Copy stream (the GPU analogue of kernel_copy, bench/stream.c:106-115): copies nbytes
 * between two device buffers `iters` times; GB/s counts the bytes read plus the bytes
 * written. Its kernel (k_copy_stream) is also the known-size reference for HBM counters.
 * The source holds the read stream's pattern and *checksum (may be NULL) is the read
 * stream's sum over the destination after the copies. */
int tf_hip_copy_stream(int device, size_t nbytes, int32_t iters, double* best_gbs, double* median_gbs,
                       uint32_t* checksum);

#ifdef __cplusplus
}
#endif
#endif /* TF_HIP_H */
