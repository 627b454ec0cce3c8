// Internal types shared by the HIP translation units of libtf_hip.so.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <vector>

#include "tf_hip.h"

namespace tfk {

constexpr int kWave = 64;        // CDNA wavefront
constexpr int kBlock = 256;      // threads per workgroup for the streaming kernels
constexpr int kWavesPerBlock = kBlock / kWave;

// One weight matrix [N rows x K] in the backend's HBM layout. The GGUF bytes are
// split into streams so that every lane step is one aligned 16-byte load:
//   Q8_0: q  = i8 [N][K]    the GGUF quants, s = f16 d [N][K/32]
//   Q4_0: q  = u8 [N][K/2]  the GGUF nibble bytes (element j low, j+16 high), s = f16 d [N][K/32]
//   Q4_1: q  = as Q4_0,     s = f16 pairs (d, m) [N][K/32]
//   Q6_K: q  = u8 [N][K/2]  low nibbles of each 32-element group (element j low, j+16 high)
//         q2 = u8 [N][K/4]  top two bits: byte j of a group holds elements j, j+8, j+16, j+24
//         s  = i8 [N][K/16] sub-block scales, s2 = f16 d [N][K/256]
//   F32:  q  = f32 [N][K];  F16: q = f16 [N][K]
// Every value the GGUF block holds is kept; only its position changes, so the bytes
// per row equal the GGUF row bytes.
struct DevMat {
    int type = -1;
    int64_t K = 0, N = 0;
    uint8_t* q = nullptr;
    uint8_t* q2 = nullptr;
    uint8_t* s = nullptr;
    uint8_t* s2 = nullptr;
    size_t gguf_bytes = 0;
    bool valid() const { return type >= 0; }
};

// Control block in device memory; the captured decode graph reads and advances it.
struct Ctl {
    int32_t pos;         // position of the token this step consumes
    int32_t att_start;   // first cache position attention covers (prefill semantics)
    int32_t mode;        // 0: token staged by the host at hist[pos], 1: argmax of the previous step
    uint32_t epoch;      // exchange epochs used so far by the persistent step kernel
    unsigned long long key;  // argmax key of the last lm_head: (ordered value << 32) | ~index
    int32_t last_token;
    int32_t err;
};

__host__ __device__ inline int32_t key_to_index(unsigned long long k) {
    return (int32_t)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull));
}

// Epilogue of a GEMV segment.
enum GemvMode : int {
    GEMV_STORE = 0,   // y[r] = acc (+ bias[r])
    GEMV_RESID = 1,   // y[r] += acc; tap[r] = y[r] when tap != nullptr
    GEMV_SILU = 2,    // paired rows: y[r] = silu(acc_gate) * acc_up
    GEMV_LOGITS = 3,  // y[r] = acc when y != nullptr; argmax folded into ctl->key
};

struct GemvSeg {
    DevMat a;            // weight (gate for GEMV_SILU)
    DevMat b;            // up matrix for GEMV_SILU
    float* y = nullptr;
    const float* bias = nullptr;
    float* tap = nullptr;
    int64_t groups = 0;  // row groups in this segment
};

constexpr int kMaxSegs = 3;

struct GemvArgs {
    GemvSeg seg[kMaxSegs];
    int n_seg = 0;
    int64_t total_groups = 0;
    int64_t K = 0;
    int type = -1;
    int mode = GEMV_STORE;
    const float* x = nullptr;       // input vector(s): n_x rows of K floats
    const float* norm_w = nullptr;  // rmsnorm weight applied to x in the prologue, or nullptr
    float eps = 0;
    Ctl* ctl = nullptr;             // GEMV_LOGITS: argmax target; bumps ctl->pos when bump_pos
    int bump_pos = 0;
    float* norm_out = nullptr;      // optional copy of the normed x (parity tap of the final norm)
};

struct AttnArgs {
    const float* q;         // [H][hd] raw (bias added, not rotated)
    const float* knew;      // [G][hd] raw, or nullptr: the cache already holds the row at pos
    const float* vnew;      // [G][hd], or nullptr as knew
    float* kc;              // this layer's K cache
    float* vc;              // this layer's V cache
    const float* rope_cos;  // [max_seq][hd/2]
    const float* rope_sin;
    float* part_o;          // [H][S][hd]
    float* part_ml;         // [H][S][2]
    float* out;             // [H][hd]
    const Ctl* ctl;
    int H, G, hd, max_seq, layout, S, rope, store_kv;
    int fixed_pos;          // >= 0: use this position instead of ctl->pos (op-level entry)
    int fixed_start;
};

// Attention splits: positions per split at least kAttnMinChunk (one LDS tile, so a
// split is one memory round), at most kAttnMaxSplits splits per kv head; one split (no
// merge launch) when max_seq <= 512.
constexpr int kAttnMinChunk = 32;
constexpr int kAttnMaxSplits = 512;
int attn_splits(int max_seq);

// ---------------------------------------------------------------- persistent step kernel
constexpr int kStepThreads = 512;  // one workgroup per CU, 8 waves

// One layer's weights and cache for the persistent step kernel (an array of these lives
// in device memory).
struct StepLayer {
    DevMat wq, wk, wv, wo, wg, wu, wd;
    const float* attn_norm;
    const float* ffn_norm;
    const float* bq;  // F32 biases or nullptr
    const float* bk;
    const float* bv;
    float* kc;        // this layer's K and V cache
    float* vc;
};

struct StepArgs {
    const StepLayer* layers;
    DevMat embd, out;          // token embedding, lm_head
    const float* out_norm;
    const float* rope_cos;     // [max_seq][hd/2]
    const float* rope_sin;
    unsigned long long* ex;    // exchange words, see step_exchange_words()
    Ctl* ctl;
    int32_t* hist;             // token per position
    float* logits;             // last token's logits, or nullptr
    float* taps;               // [L+1][D] per-layer outputs of the last token, or nullptr
    int n_layer, D, F, H, G, hd, max_seq, layout;
    float eps;
    int n_tokens;              // tokens this launch runs
    int greedy;                // 0: tokens from hist (prefill, decode); 1: each token is the previous argmax
    int lm_every;              // 1: lm_head for every token; 0: for the last one only (prefill)
    int att_start;             // first cache position attention covers (0, or the prefill chunk's start)
    int stage_lds;             // ffn_down staged in LDS (step_stage_lds): 1 a row per wave, 2 split over K per workgroup
    int split;                 // > 0: split attention on the trailing workgroups, splits per kv head (step_split)
    int split_all;             // > 0: splits per kv head when every workgroup splits (step_split_all)
    int split_all_from;        // spans longer than this use split_all (step_split_all_from)
    int split_from;            // spans (positions attended) up to this attend on one workgroup per kv head
};

// ---------------------------------------------------------------- prefill on the matrix cores
// Rows (tokens) of a prefill GEMM workgroup tile; activation buffers are padded to it.
constexpr int kPfTileM = 64;
// Rows per prefill chunk: longer prompts run in chunks whose attention covers the
// prompt so far through the cache. A 4096-token prompt in one chunk instead of two of 2048
// prefills 12 % faster (Qwen2.5-1.5B shape: the causal triangle's short query blocks fill
// CUs that the long ones leave, and the GEMMs get twice the row tiles).
constexpr int kPfChunk = 4096;

__host__ __device__ inline int64_t kv_offset(int layout, int G, int max_seq, int hd, int g, int p) {
    return layout == TF_HIP_KV_HEAD_MAJOR ? ((int64_t)g * max_seq + p) * hd : ((int64_t)p * G + g) * hd;
}

// One weight matrix of a prefill GEMM and where its output columns go.
struct PfSeg {
    DevMat w;                     // weight (gate for GEMV_SILU), read in its HBM layout
    DevMat w2;                    // up matrix for GEMV_SILU, w's format
    float* y = nullptr;           // output rows of ldy floats
    int64_t ldy = 0;
    const float* bias = nullptr;  // F32 bias added to the output (GEMV_STORE)
    int sub0 = 0;                 // first 16-column output subtile of this segment
};

// C[M x N] = A[M x K] . W^T over the matrix cores. A arrives as fp16 pairs hi + lo whose
// sum is each row times a power of two (rs holds the inverse), see launch_pf_split.
struct PfGemmArgs {
    const uint16_t* xa = nullptr;  // [Mpad/16][K/32][hi, lo][64][8] fp16 (fragment order)
    const float* rs = nullptr;     // [Mpad] row scales
    int K = 0, M = 0, Mpad = 0;
    PfSeg seg[3];
    int n_seg = 0;
    int n_sub = 0;                 // 16-column output subtiles over all segments
    int mode = GEMV_STORE;         // GEMV_STORE, GEMV_RESID or GEMV_SILU
    float* tap = nullptr;          // GEMV_RESID: copy of output row tap_row
    int tap_row = -1;
    float* part = nullptr;         // optional workspace for split-K partial sums (GEMV_STORE, GEMV_RESID)
    size_t part_floats = 0;
    int ks = 1;                    // K slices (set by launch_pf_gemm)
    // Work the split-K reduce can take over from the kernel that follows the GEMM
    // (launch_pf_gemm reports through *fused whether it did):
    // GEMV_RESID over one segment, split_xa set: the split of every updated row
    // (launch_pf_split of the output rows, rmsnorm with split_w when given); GEMV_SILU with
    // K split, split_xa set: the split of the silu * up rows, which are then not stored
    uint16_t* split_xa = nullptr;
    float* split_rs = nullptr;
    const float* split_w = nullptr;
    float split_eps = 0.0f;
    // GEMV_STORE of the q, k and v segments, rope_cos set: launch_pf_rope_store of the rows
    // (q rotated into its segment's rows, k rotated and v into the cache at pos0 + row)
    const float* rope_cos = nullptr;
    const float* rope_sin = nullptr;
    float* kc = nullptr;
    float* vc = nullptr;
    int pos0 = 0, n_head = 0, n_kv = 0, hd = 0, kv_layout = 0, max_seq = 0;
};

// Q8_0, Q4_0, Q4_1, F16, F32 or Q6_K (K % 256 == 0) with K % 64 == 0 and N % 16 == 0; the
// matrices of one launch_pf_gemm share one format.
bool pf_gemm_supported(int type, int64_t K, int64_t N);
// xa needs Mpad * K * 2 halves, rs Mpad floats.
hipError_t launch_pf_split(const float* x, int64_t ldx, const float* norm_w, float eps, int K, int M, int Mpad,
                           uint16_t* xa, float* rs, hipStream_t st);
hipError_t launch_pf_gemm(const PfGemmArgs& a, hipStream_t st, bool* fused = nullptr);
hipError_t launch_embed_rows(const DevMat& emb, const int32_t* tok, int n, float* x, int D, hipStream_t st);
hipError_t launch_pf_rope_store(float* qkv, int64_t ld, int n, int H, int G, int hd, const float* rope_cos,
                                const float* rope_sin, int pos0, float* kc, float* vc, int layout, int max_seq,
                                hipStream_t st);
bool pf_attn_supported(int hd, int n_rep);
// Workspace of launch_pf_attn for attention over n_keys positions: the packed key/value
// tile records.
size_t pf_attn_ws_bytes(int hd, int G, int n_keys);
hipError_t launch_pf_attn(const float* q, int64_t ldq, const float* kc, const float* vc, int layout, int H, int G,
                          int hd, int max_seq, int n, int pos0, int att_start, float* out, int64_t ldo, void* ws,
                          size_t ws_bytes, hipStream_t st);
hipError_t launch_pf_tail(Ctl* ctl, int pos_last, const int32_t* hist, const float* xrow, float* x, int D,
                          hipStream_t st);

// Exchange words of the step kernel; split: the larger of its two splits per kv head.
size_t step_exchange_words(int D, int F, int H, int G, int hd, int n_wg, int split);
// Splits per kv head of the step kernel's attention for caches longer than 512 positions,
// or 0 when the model's shape does not allow it: step_split on the trailing workgroups
// (the others stream wo's and the FFN's weights meanwhile), step_split_all on every
// workgroup (for long spans).
int step_split(int D, int F, int H, int G, int hd, int n_wg);
int step_split_all(int D, int F, int H, int G, int hd, int n_wg);
// The span (cache positions attended) past which every workgroup splits instead.
int step_split_all_from(int H, int G, int hd, int split);
size_t step_lds_bytes(int n_layer, int D, int F, int H, int G, int hd, int n_wg, int stage_lds);
// Which weight rows the step kernel stages in LDS ahead of their phase (bits of
// StepArgs::stage_lds): the ffn_down rows (bit 0) for Q8_0 layers with at most one row per
// wave and the LDS for them. (Staging the next layer's QKV rows as well was measured twice:
// issued with the ffn_down rows, the exchange that waits behind their loads loses what the
// QKV phase gains; issued in the down phase once its input is in, as loads the compiler does
// not wait for, the down rows' exchange writes go out behind them: Llama-3.2-1B shape
// 0.502 -> 0.527, Qwen2.5-0.5B 0.591 -> 0.616 ms per token.)
int step_stage_lds(int type_layers, int n_layer, int D, int F, int H, int G, int hd, int n_wg);
// true when the model's formats, head size and query heads per kv head (n_rep) have a
// compiled step kernel.
bool step_supported(int type_layers, int type_out, int hd, int n_rep);
// The second format the step kernel for layer format tl takes for wo and ffn_down (tl when
// there is none).
int step_alt_type(int tl);
hipError_t launch_step(const StepArgs& a, int type_layers, int type_out, int n_wg, hipStream_t st);
// the Q8_0 builds with ffn_down split over K (stage_lds 2)
hipError_t launch_step_split(const StepArgs& a, int n_wg, hipStream_t st);

// Launchers (k_*.hip).
hipError_t launch_gemv(const GemvArgs& a, int rows_per_wave, hipStream_t st);
int64_t gemv_groups(int64_t n_rows, int rows_per_wave);
size_t gemv_lds_bytes(int64_t K);
hipError_t launch_attn_decode(const AttnArgs& a, hipStream_t st);
hipError_t launch_embed(const DevMat& emb, float* x, Ctl* ctl, int32_t* hist, int D, hipStream_t st);
hipError_t launch_dequant_rows(const DevMat& m, int64_t row0, int64_t nrows, float* out, hipStream_t st);
hipError_t launch_repack(int type, const uint8_t* raw, int64_t K, int64_t N, DevMat& m, hipStream_t st);
hipError_t launch_rmsnorm_rows(const float* x, const float* w, int n, int rows, float eps, float* out,
                               hipStream_t st);
// Temperature / nucleus sampling (k_sample.hip): device workspace bytes for n logits, and
// the launches that sample one token into d_token (optional sorted order and final
// probabilities into d_sorted_idx / d_probs, n each).
size_t sample_work_bytes(int n);
hipError_t launch_sample(const float* logits, int n, float temperature, float top_p, float r, void* work,
                         size_t work_bytes, int32_t* d_token, int32_t* d_sorted_idx, float* d_probs, hipStream_t st);
hipError_t launch_rope_rows(float* x, int seq, int n_heads, int hd, int pos0, const float* cos_tab,
                            const float* sin_tab, hipStream_t st);
hipError_t launch_argmax(const float* x, int n, Ctl* ctl, hipStream_t st);
// The read and copy streams (k_misc.hip): buffers filled by launch_fill_stream hold 32-bit
// word i = i * kStreamMul, and k_read_stream writes one integer partial sum per wave.
constexpr uint32_t kStreamMul = 0x9E3779B1u;
hipError_t launch_copy_stream(uint4* dst, const uint4* src, size_t n4, int blocks, hipStream_t st);
hipError_t launch_read_stream(const uint4* p, size_t n4, uint32_t* out, int blocks, hipStream_t st);
hipError_t launch_fill_stream(uint4* p, size_t n4, int blocks, hipStream_t st);
int device_cu_count();

}  // namespace tfk
