// libtf_hip: the C ABI of include/tf_hip.h over the gfx950 kernels.
//
// A context owns the weights (repacked into the DevMat layout), the fp32 KV cache,
// the activations and one captured hipGraph for a decode step. The graph reads the
// token and position from the device control block (Ctl), so the same graph serves
// decode (token staged in the token history), prefill (all prompt tokens staged,
// replayed once per token with attention limited to the prompt, as attn_prefill
// does) and the greedy loop (token = previous argmax, no host round trip).
#include <algorithm>
#include <cstdio>
#include <mutex>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "formats.hpp"
#include "tf_internal.hpp"

using namespace tfk;

namespace {

constexpr int kNumClasses = 7;  // embed, qkv, attention, wo, gate/up, down, lm_head
const char* const kClassNames[kNumClasses] = {"embed", "qkv_gemv", "attention", "wo_gemv",
                                              "gateup_gemv", "down_gemv", "lmhead_gemv"};

// One workgroup per kv head attends two 32-position tiles faster than a split's extra merge
// hand-off; past that its tiles cost more (Llama-3.2-1B shape on MI355X: 0.533 vs 0.544 ms
// per token at spans 7-38, 1.015 vs 0.557 at spans 301-428). One workgroup per kv head
// attends at most 512 positions.
constexpr int kSplitFromDefault = 64;
constexpr int kSplitFromMax = 512;

struct Prof {
    std::vector<hipEvent_t> ev;  // pairs per launch
    std::vector<int> cls;
    std::vector<double> bytes;
};

}  // namespace

struct tf_hip_ctx {
    int device = 0;
    hipStream_t st = nullptr;
    tf_hip_hparams hp{};
    int H = 0, KVd = 0;  // n_head*head_dim, n_kv_head*head_dim
    std::vector<DevMat> mats;
    std::vector<float*> vecs;
    std::vector<int64_t> vec_len;
    std::vector<void*> allocs;
    float* kc = nullptr;
    float* vc = nullptr;
    size_t kv_layer = 0;  // floats per layer
    float* rope_cos = nullptr;
    float* rope_sin = nullptr;
    bool rope_set = false;
    float *x = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *att = nullptr, *h = nullptr;
    float *logits = nullptr, *taps = nullptr, *part_o = nullptr, *part_ml = nullptr;
    Ctl* ctl = nullptr;
    Ctl* ctl_host = nullptr;      // pinned staging
    int32_t* hist = nullptr;      // device token per position
    int32_t* tok_host = nullptr;  // pinned staging [max_seq]
    int S = 1;                    // attention splits per kv head
    int pos = 0;
    bool have_logits = false;
    void* sample_work = nullptr;      // tf_hip_sample: sort buffers, probabilities, radix-sort scratch
    size_t sample_bytes = 0;
    int32_t* d_sampled = nullptr;     // the sampled token
    Ctl* sample_ctl = nullptr;        // argmax of a greedy tf_hip_sample
    hipGraph_t graph = nullptr;
    hipGraphExec_t gexec = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    float last_ms = 0;
    int last_steps = 0;
    const char* last_name = "decode_graph";  // what the last timed call ran
    // persistent step kernel (k_step.hpp)
    int path_opt = TF_HIP_PATH_STEP;  // requested decode path
    int step_state = -1;              // -1 undecided, 0 graph path, 1 step kernel ready
    int step_tl = -1, step_to = -1, n_wg = 0;
    int step_split = 0, step_split_all = 0;  // the step kernel's attention splits (step_split*)
    int split_all_from = -1;                  // tf_hip_set_split_all_from (< 0: step_split_all_from)
    int split_from = kSplitFromDefault;       // tf_hip_set_split_from: spans up to this attend unsplit
    StepLayer* d_layers = nullptr;
    bool coop_refused = false;  // the GPU refused the step kernel's cooperative launch: graph path from then on
    int refuse_coop = 0;        // test hook: this many more step launches report a refusal
    unsigned long long* ex = nullptr;
    size_t ex_words = 0;
    uint32_t epoch = 0;               // exchange epochs consumed (mirrors ctl->epoch)
    // prefill on the matrix cores (k_prefill.hip)
    int pf_opt = TF_HIP_PREFILL_MFMA;  // requested prefill path
    int pf_state = -1;                 // -1 undecided, 0 per-token path, 1 matrix-core path ready
    int pf_cap = 0;                    // rows per prefill chunk (multiple of kPfTileM)
    float *px = nullptr, *pqkv = nullptr, *patt = nullptr, *ph = nullptr, *prs = nullptr;
    uint16_t* pxa = nullptr;            // activation fragments (hi, lo) of one chunk
    float* ppart = nullptr;             // split-K partial sums of the prefill GEMMs
    size_t ppart_floats = 0;
    void* pattn_ws = nullptr;           // packed key/value tiles of prefill attention
    size_t pattn_ws_bytes = 0;
    std::string err;
};

namespace {

int fail(tf_hip_ctx* c, int code, const std::string& msg) {
    if (c) c->err = msg;
    return code;
}

#define HIPCHK(ctx, call)                                                                      \
    do {                                                                                       \
        hipError_t e_ = (call);                                                                \
        if (e_ != hipSuccess)                                                                  \
            return fail(ctx, e_ == hipErrorOutOfMemory ? TF_HIP_ENOMEM : TF_HIP_EDEVICE,      \
                        std::string(#call) + ": " + hipGetErrorString(e_));                    \
    } while (0)

template <typename T>
int dalloc(tf_hip_ctx* c, T** p, size_t bytes) {
    void* d = nullptr;
    const hipError_t e = hipMalloc(&d, bytes ? bytes : 16);
    if (e != hipSuccess)
        return fail(c, TF_HIP_ENOMEM, "hipMalloc(" + std::to_string(bytes) + "): " + hipGetErrorString(e));
    c->allocs.push_back(d);
    *p = (T*)d;
    return 0;
}

size_t blck_bytes(int t) {
    switch (t) {
        case TF_HIP_TYPE_F32: return 4;
        case TF_HIP_TYPE_F16: return 2;
        case TF_HIP_TYPE_Q4_0: return 18;
        case TF_HIP_TYPE_Q4_1: return 20;
        case TF_HIP_TYPE_Q8_0: return 34;
        case TF_HIP_TYPE_Q6_K: return 210;
    }
    return 0;
}
int blck_elems(int t) {
    switch (t) {
        case TF_HIP_TYPE_Q4_0:
        case TF_HIP_TYPE_Q4_1:
        case TF_HIP_TYPE_Q8_0: return 32;
        case TF_HIP_TYPE_Q6_K: return 256;
        case TF_HIP_TYPE_F32:
        case TF_HIP_TYPE_F16: return 1;
    }
    return 0;
}

// Row length constraints of the backend layout (16-byte lane steps).
bool row_ok(int t, int64_t K) {
    if (blck_elems(t) == 0 || K <= 0) return false;
    switch (t) {
        case TF_HIP_TYPE_F32: return K % 4 == 0;
        case TF_HIP_TYPE_F16: return K % 8 == 0;
        case TF_HIP_TYPE_Q6_K: return K % 256 == 0;
        default: return K % 32 == 0;
    }
}

size_t gguf_nbytes(int t, int64_t K, int64_t N) { return (size_t)N * (size_t)(K / blck_elems(t)) * blck_bytes(t); }

// Allocates the streams of m and converts the GGUF bytes (already on the device) into them.
hipError_t make_devmat(int t, int64_t K, int64_t N, const uint8_t* d_raw, DevMat& m, std::vector<void*>& owned,
                       hipStream_t st) {
    m.type = t;
    m.K = K;
    m.N = N;
    m.gguf_bytes = gguf_nbytes(t, K, N);
    auto al = [&](uint8_t** p, size_t n) -> hipError_t {
        void* d = nullptr;
        hipError_t e = hipMalloc(&d, n ? n : 16);
        if (e == hipSuccess) owned.push_back(d);
        *p = (uint8_t*)d;
        return e;
    };
    hipError_t e = hipSuccess;
    switch (t) {
        case TF_HIP_TYPE_F32:
        case TF_HIP_TYPE_F16:
            if ((e = al(&m.q, m.gguf_bytes)) != hipSuccess) return e;
            return hipMemcpyAsync(m.q, d_raw, m.gguf_bytes, hipMemcpyDeviceToDevice, st);
        case TF_HIP_TYPE_Q8_0:
            if ((e = al(&m.q, (size_t)N * K)) != hipSuccess) return e;
            if ((e = al(&m.s, (size_t)N * (K / 32) * 2)) != hipSuccess) return e;
            break;
        case TF_HIP_TYPE_Q4_0:
            if ((e = al(&m.q, (size_t)N * K / 2)) != hipSuccess) return e;
            if ((e = al(&m.s, (size_t)N * (K / 32) * 2)) != hipSuccess) return e;
            break;
        case TF_HIP_TYPE_Q4_1:
            if ((e = al(&m.q, (size_t)N * K / 2)) != hipSuccess) return e;
            if ((e = al(&m.s, (size_t)N * (K / 32) * 4)) != hipSuccess) return e;
            break;
        case TF_HIP_TYPE_Q6_K:
            if ((e = al(&m.q, (size_t)N * K / 2)) != hipSuccess) return e;
            if ((e = al(&m.q2, (size_t)N * K / 4)) != hipSuccess) return e;
            if ((e = al(&m.s, (size_t)N * (K / 16))) != hipSuccess) return e;
            if ((e = al(&m.s2, (size_t)N * (K / 256) * 2)) != hipSuccess) return e;
            break;
        default: return hipErrorInvalidValue;
    }
    return launch_repack(t, d_raw, K, N, m, st);
}

// Rows per wavefront: two (swept on MI355X for the decode shapes); one for matrices
// too short to give every CU a group.
int pick_rows(int64_t n_rows) { return n_rows >= 2LL * kWavesPerBlock * device_cu_count() ? 2 : 1; }

void add_seg(GemvArgs& a, const DevMat& m, float* y, const float* bias, float* tap, int R) {
    GemvSeg& s = a.seg[a.n_seg++];
    s.a = m;
    s.y = y;
    s.bias = bias;
    s.tap = tap;
    s.groups = gemv_groups(m.N, R);
    a.total_groups += s.groups;
}

const DevMat& mat(const tf_hip_ctx* c, int slot) { return c->mats[(size_t)slot]; }
const float* vec(const tf_hip_ctx* c, int slot) { return c->vecs[(size_t)slot]; }

const DevMat& output_mat(const tf_hip_ctx* c) {
    return mat(c, TF_HIP_SLOT_OUTPUT).valid() ? mat(c, TF_HIP_SLOT_OUTPUT) : mat(c, TF_HIP_SLOT_TOKEN_EMBD);
}

int check_ready(tf_hip_ctx* c) {
    auto need_m = [&](int slot, const char* what) -> bool {
        if (!mat(c, slot).valid()) {
            c->err = std::string("tensor not uploaded: ") + what;
            return false;
        }
        return true;
    };
    auto need_v = [&](int slot, const char* what) -> bool {
        if (!vec(c, slot)) {
            c->err = std::string("tensor not uploaded: ") + what;
            return false;
        }
        return true;
    };
    if (!need_m(TF_HIP_SLOT_TOKEN_EMBD, "token_embd.weight") || !need_v(TF_HIP_SLOT_OUTPUT_NORM, "output_norm.weight"))
        return TF_HIP_ESTATE;
    for (int l = 0; l < c->hp.n_layer; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        if (!need_v(TF_HIP_SLOT_LAYER(l, TF_HIP_LAYER_ATTN_NORM), (p + "attn_norm").c_str()) ||
            !need_m(TF_HIP_SLOT_LAYER(l, TF_HIP_LAYER_Q), (p + "attn_q").c_str()) ||
            !need_m(TF_HIP_SLOT_LAYER(l, TF_HIP_LAYER_K), (p + "attn_k").c_str()) ||
            !need_m(TF_HIP_SLOT_LAYER(l, TF_HIP_LAYER_V), (p + "attn_v").c_str()) ||
            !need_m(TF_HIP_SLOT_LAYER(l, TF_HIP_LAYER_O), (p + "attn_output").c_str()) ||
            !need_v(TF_HIP_SLOT_LAYER(l, TF_HIP_LAYER_FFN_NORM), (p + "ffn_norm").c_str()) ||
            !need_m(TF_HIP_SLOT_LAYER(l, TF_HIP_LAYER_GATE), (p + "ffn_gate").c_str()) ||
            !need_m(TF_HIP_SLOT_LAYER(l, TF_HIP_LAYER_UP), (p + "ffn_up").c_str()) ||
            !need_m(TF_HIP_SLOT_LAYER(l, TF_HIP_LAYER_DOWN), (p + "ffn_down").c_str()))
            return TF_HIP_ESTATE;
    }
    if (!c->rope_set) {
        c->err = "RoPE table not set";
        return TF_HIP_ESTATE;
    }
    return 0;
}

// Launch one kernel, bracketed by events when profiling.
struct Launcher {
    tf_hip_ctx* c;
    Prof* prof;
    hipError_t err = hipSuccess;
    template <typename Fn>
    void run(int cls, double bytes, Fn fn) {
        if (err != hipSuccess) return;
        hipEvent_t a = nullptr, b = nullptr;
        if (prof) {
            (void)hipEventCreate(&a);
            (void)hipEventCreate(&b);
            (void)hipEventRecord(a, c->st);
        }
        err = fn();
        if (prof) {
            (void)hipEventRecord(b, c->st);
            prof->ev.push_back(a);
            prof->ev.push_back(b);
            prof->cls.push_back(cls);
            prof->bytes.push_back(bytes);
        }
    }
};

// Final rmsnorm and lm_head of c->x (model.cpp:189-193, 204-206): logits, the argmax
// into ctl->key, the normed row into the last tap, and ctl->pos advanced by one.
hipError_t launch_lm_head(tf_hip_ctx* c) {
    const DevMat& wout = output_mat(c);
    const int R = pick_rows(wout.N);
    GemvArgs a;
    a.type = wout.type;
    a.K = c->hp.n_embd;
    a.mode = GEMV_LOGITS;
    a.x = c->x;
    a.norm_w = vec(c, TF_HIP_SLOT_OUTPUT_NORM);
    a.eps = c->hp.rms_eps;
    a.norm_out = c->taps + (size_t)c->hp.n_layer * c->hp.n_embd;
    a.ctl = c->ctl;
    a.bump_pos = 1;
    add_seg(a, wout, c->logits, nullptr, nullptr, R);
    return launch_gemv(a, R, c->st);
}

// One decode step (model.cpp:197-208) on the context stream.
// pos/att_start only size the profile's byte counts; the kernels read them from Ctl.
hipError_t enqueue_step(tf_hip_ctx* c, Prof* prof, int pos = 0, int att_start = 0) {
    const tf_hip_hparams& hp = c->hp;
    const int D = hp.n_embd, F = hp.n_ff;
    Launcher L{c, prof};
    const DevMat& emb = mat(c, TF_HIP_SLOT_TOKEN_EMBD);
    L.run(0, (double)emb.gguf_bytes / emb.N, [&] { return launch_embed(emb, c->x, c->ctl, c->hist, D, c->st); });
    for (int l = 0; l < hp.n_layer; ++l) {
        auto M = [&](int kind) -> const DevMat& { return mat(c, TF_HIP_SLOT_LAYER(l, kind)); };
        auto V = [&](int kind) { return vec(c, TF_HIP_SLOT_LAYER(l, kind)); };
        // Q, K, V (+bias): one launch when the three share a format
        {
            const DevMat& wq = M(TF_HIP_LAYER_Q);
            const DevMat& wk = M(TF_HIP_LAYER_K);
            const DevMat& wv = M(TF_HIP_LAYER_V);
            const int R = pick_rows(wq.N + wk.N + wv.N);
            const DevMat* ms[3] = {&wq, &wk, &wv};
            float* ys[3] = {c->q, c->k, c->v};
            const float* bs[3] = {V(TF_HIP_LAYER_BQ), V(TF_HIP_LAYER_BK), V(TF_HIP_LAYER_BV)};
            int i = 0;
            while (i < 3) {
                GemvArgs a;
                a.type = ms[i]->type;
                a.K = D;
                a.mode = GEMV_STORE;
                a.x = c->x;
                a.norm_w = V(TF_HIP_LAYER_ATTN_NORM);
                a.eps = hp.rms_eps;
                // the first launch also reads the norm weights; each segment its bias
                double bytes = i == 0 ? 4.0 * D : 0.0;
                while (i < 3 && ms[i]->type == a.type) {
                    add_seg(a, *ms[i], ys[i], bs[i], nullptr, R);
                    bytes += (double)ms[i]->gguf_bytes + (bs[i] ? 4.0 * (double)ms[i]->N : 0.0);
                    ++i;
                }
                L.run(1, bytes, [&] { return launch_gemv(a, R, c->st); });
            }
        }
        {
            AttnArgs a{};
            a.q = c->q;
            a.knew = c->k;
            a.vnew = c->v;
            a.kc = c->kc + (size_t)l * c->kv_layer;
            a.vc = c->vc + (size_t)l * c->kv_layer;
            a.rope_cos = c->rope_cos;
            a.rope_sin = c->rope_sin;
            a.part_o = c->part_o;
            a.part_ml = c->part_ml;
            a.out = c->att;
            a.ctl = c->ctl;
            a.H = hp.n_head;
            a.G = hp.n_kv_head;
            a.hd = hp.head_dim;
            a.max_seq = hp.max_seq;
            a.layout = hp.kv_layout;
            a.S = c->S;
            a.rope = 1;
            a.store_kv = 1;
            a.fixed_pos = -1;
            a.fixed_start = 0;
            // K and V rows of positions [att_start, pos] and the new row written
            const double kv_bytes = (double)hp.n_kv_head * hp.head_dim * 4.0 * 2.0 * (pos - att_start + 2);
            L.run(2, kv_bytes, [&] { return launch_attn_decode(a, c->st); });
        }
        {
            const DevMat& wo = M(TF_HIP_LAYER_O);
            const int R = pick_rows(wo.N);
            GemvArgs a;
            a.type = wo.type;
            a.K = c->H;
            a.mode = GEMV_RESID;
            a.x = c->att;
            add_seg(a, wo, c->x, nullptr, nullptr, R);
            L.run(3, (double)wo.gguf_bytes, [&] { return launch_gemv(a, R, c->st); });
        }
        {
            const DevMat& wg = M(TF_HIP_LAYER_GATE);
            const DevMat& wu = M(TF_HIP_LAYER_UP);
            if (wg.type == wu.type) {
                const int R = pick_rows(wg.N);
                GemvArgs a;
                a.type = wg.type;
                a.K = D;
                a.mode = GEMV_SILU;
                a.x = c->x;
                a.norm_w = V(TF_HIP_LAYER_FFN_NORM);
                a.eps = hp.rms_eps;
                add_seg(a, wg, c->h, nullptr, nullptr, R);
                a.seg[0].b = wu;
                L.run(4, (double)(wg.gguf_bytes + wu.gguf_bytes) + 4.0 * D, [&] { return launch_gemv(a, R, c->st); });
            } else {
                L.err = hipErrorInvalidValue;  // rejected at upload; unreachable
            }
        }
        {
            const DevMat& wd = M(TF_HIP_LAYER_DOWN);
            const int R = pick_rows(wd.N);
            GemvArgs a;
            a.type = wd.type;
            a.K = F;
            a.mode = GEMV_RESID;
            a.x = c->h;
            add_seg(a, wd, c->x, nullptr, c->taps + (size_t)l * D, R);
            L.run(5, (double)wd.gguf_bytes, [&] { return launch_gemv(a, R, c->st); });
        }
    }
    {
        const DevMat& wout = output_mat(c);
        L.run(6, (double)wout.gguf_bytes + 4.0 * D, [&] { return launch_lm_head(c); });
    }
    return L.err;
}

int ensure_graph(tf_hip_ctx* c) {
    if (c->gexec) return 0;
    int rc = check_ready(c);
    if (rc) return rc;
    HIPCHK(c, hipStreamBeginCapture(c->st, hipStreamCaptureModeThreadLocal));
    const hipError_t e = enqueue_step(c, nullptr);
    hipGraph_t g = nullptr;
    const hipError_t e2 = hipStreamEndCapture(c->st, &g);
    if (e != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return fail(c, TF_HIP_EDEVICE, std::string("decode step launch: ") + hipGetErrorString(e));
    }
    if (e2 != hipSuccess) return fail(c, TF_HIP_EDEVICE, std::string("hipStreamEndCapture: ") + hipGetErrorString(e2));
    c->graph = g;
    HIPCHK(c, hipGraphInstantiate(&c->gexec, c->graph, nullptr, nullptr, 0));
    return 0;
}

// Decides once, after every tensor is uploaded, whether the persistent step kernel runs
// this model: one format for all layer matrices (wo and ffn_down may also have the
// kernel's second format, step_alt_type: Q4_1 beside Q4_0), the embedding in the lm_head's
// format, a compiled (format, head size) combination, cooperative launch, and inputs within the
// kernel's per-thread capacities. Caches longer than 512 positions split each layer's
// attention over workgroups (step_split, step_split_all). Returns 1 (step kernel), 0
// (graph) or < 0.
int ensure_step(tf_hip_ctx* c) {
    if (c->path_opt == TF_HIP_PATH_GRAPH || c->coop_refused) return 0;
    if (c->step_state >= 0) return c->step_state;
    int rc = check_ready(c);
    if (rc) return rc;
    c->step_state = 0;
    const tf_hip_hparams& p = c->hp;
    const int tl = mat(c, TF_HIP_SLOT_LAYER(0, TF_HIP_LAYER_Q)).type;
    const int kinds[7] = {TF_HIP_LAYER_Q,    TF_HIP_LAYER_K,  TF_HIP_LAYER_V,   TF_HIP_LAYER_O,
                          TF_HIP_LAYER_GATE, TF_HIP_LAYER_UP, TF_HIP_LAYER_DOWN};
    const int ta = step_alt_type(tl);  // wo and ffn_down may also have this format
    for (int l = 0; l < p.n_layer; ++l)
        for (int k : kinds) {
            const int t = mat(c, TF_HIP_SLOT_LAYER(l, k)).type;
            const bool alt_ok = k == TF_HIP_LAYER_O || k == TF_HIP_LAYER_DOWN;
            if (t != tl && !(alt_ok && t == ta)) return 0;
        }
    const DevMat& out = output_mat(c);
    if (mat(c, TF_HIP_SLOT_TOKEN_EMBD).type != out.type ||
        !step_supported(tl, out.type, p.head_dim, p.n_head / p.n_kv_head))
        return 0;
    int coop = 0;
    if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, c->device) != hipSuccess || !coop) return 0;
    const int n_wg = device_cu_count();
    const int n_rep = p.n_head / p.n_kv_head;
    if (n_wg < 2 * p.n_kv_head || p.n_embd + n_wg > 4096 || p.n_ff > 10240 || 2 * n_wg > 1024 ||
        (n_rep + 2) * p.head_dim > 4096 || p.n_head * p.head_dim > 4096)
        return 0;
    // attention split over workgroups for tokens past StepArgs::split_from positions
    // (required past 512: one workgroup per kv head attends at most that many)
    const int split = step_split(p.n_embd, p.n_ff, p.n_head, p.n_kv_head, p.head_dim, n_wg);
    if (p.max_seq > 512 && !split) return 0;
    std::vector<StepLayer> tab((size_t)p.n_layer);
    for (int l = 0; l < p.n_layer; ++l) {
        auto M = [&](int k) -> const DevMat& { return mat(c, TF_HIP_SLOT_LAYER(l, k)); };
        auto V = [&](int k) { return vec(c, TF_HIP_SLOT_LAYER(l, k)); };
        StepLayer& t = tab[(size_t)l];
        t.wq = M(TF_HIP_LAYER_Q);
        t.wk = M(TF_HIP_LAYER_K);
        t.wv = M(TF_HIP_LAYER_V);
        t.wo = M(TF_HIP_LAYER_O);
        t.wg = M(TF_HIP_LAYER_GATE);
        t.wu = M(TF_HIP_LAYER_UP);
        t.wd = M(TF_HIP_LAYER_DOWN);
        t.attn_norm = V(TF_HIP_LAYER_ATTN_NORM);
        t.ffn_norm = V(TF_HIP_LAYER_FFN_NORM);
        t.bq = V(TF_HIP_LAYER_BQ);
        t.bk = V(TF_HIP_LAYER_BK);
        t.bv = V(TF_HIP_LAYER_BV);
        t.kc = c->kc + (size_t)l * c->kv_layer;
        t.vc = c->vc + (size_t)l * c->kv_layer;
    }
    const int split_all =
        split ? step_split_all(p.n_embd, p.n_ff, p.n_head, p.n_kv_head, p.head_dim, n_wg) : 0;
    c->step_split_all = split_all;
    const size_t words = step_exchange_words(p.n_embd, p.n_ff, p.n_head, p.n_kv_head, p.head_dim, n_wg,
                                             split > split_all ? split : split_all);
    if ((rc = dalloc(c, &c->d_layers, tab.size() * sizeof(StepLayer))) || (rc = dalloc(c, &c->ex, words * 8)))
        return rc;
    HIPCHK(c, hipMemcpy(c->d_layers, tab.data(), tab.size() * sizeof(StepLayer), hipMemcpyHostToDevice));
    HIPCHK(c, hipMemset(c->ex, 0, words * 8));  // epoch 0 is never used
    c->ex_words = words;
    c->step_tl = tl;
    c->step_to = out.type;
    c->n_wg = n_wg;
    c->step_split = split;
    c->step_state = 1;
    return 1;
}

// Exchange words carry 32-bit epochs, P per token, and a launch of n tokens uses c->epoch +
// 1 .. c->epoch + n P. Before that range would pass 2^32 (about 40 M tokens of the 1B shape)
// the words are cleared and the count starts again at 0, so no word left from before can
// carry an epoch a reader expects.
int epoch_guard(tf_hip_ctx* c, int n) {
    const uint64_t P = 6ull * (uint64_t)c->hp.n_layer + 8ull;
    if ((uint64_t)c->epoch + (uint64_t)n * P >= 0xFFFFFFFFull) {
        HIPCHK(c, hipStreamSynchronize(c->st));
        HIPCHK(c, hipMemsetAsync(c->ex, 0, c->ex_words * 8, c->st));
        c->epoch = 0;
        c->ctl_host->epoch = 0;
        HIPCHK(c, hipMemcpyAsync((char*)c->ctl + offsetof(Ctl, epoch), (char*)c->ctl_host + offsetof(Ctl, epoch),
                                 sizeof(uint32_t), hipMemcpyHostToDevice, c->st));
    }
    return 0;
}

// run_step's result when the GPU refused the cooperative launch: nothing ran. A second
// process on a GPU whose cooperative-launch resource another process holds gets
// hipErrorIllegalState (measured on MI355X); a grid that no longer fits, the others.
constexpr int kStepRefused = 1;
bool coop_refusal(hipError_t e) {
    return e == hipErrorIllegalState || e == hipErrorCooperativeLaunchTooLarge || e == hipErrorLaunchOutOfResources ||
           e == hipErrorNotSupported;
}

// n tokens through the persistent step kernel, from position c->pos. Returns 0,
// kStepRefused (the context then takes the graph path from now on) or < 0.
int run_step(tf_hip_ctx* c, int n, int greedy, int lm_every, int att_start) {
    const tf_hip_hparams& p = c->hp;
    StepArgs a{};
    a.layers = c->d_layers;
    a.embd = mat(c, TF_HIP_SLOT_TOKEN_EMBD);
    a.out = output_mat(c);
    a.out_norm = vec(c, TF_HIP_SLOT_OUTPUT_NORM);
    a.rope_cos = c->rope_cos;
    a.rope_sin = c->rope_sin;
    a.ex = c->ex;
    a.ctl = c->ctl;
    a.hist = c->hist;
    a.logits = c->logits;
    a.taps = c->taps;
    a.n_layer = p.n_layer;
    a.D = p.n_embd;
    a.F = p.n_ff;
    a.H = p.n_head;
    a.G = p.n_kv_head;
    a.hd = p.head_dim;
    a.max_seq = p.max_seq;
    a.layout = p.kv_layout;
    a.eps = p.rms_eps;
    a.n_tokens = n;
    a.greedy = greedy;
    a.lm_every = lm_every;
    a.att_start = att_start;
    a.stage_lds = step_stage_lds(c->step_tl, p.n_layer, p.n_embd, p.n_ff, p.n_head, p.n_kv_head, p.head_dim, c->n_wg);
    a.split = c->step_split;
    a.split_all = c->step_split_all;
    a.split_from = c->split_from;
    a.split_all_from = c->split_all_from >= 0 ? c->split_all_from
                                              : step_split_all_from(p.n_head, p.n_kv_head, p.head_dim, c->step_split);
    int rc = epoch_guard(c, n);
    if (rc) return rc;
    hipError_t e;
    if (c->refuse_coop > 0) {
        --c->refuse_coop;
        e = hipErrorCooperativeLaunchTooLarge;
    } else {
        e = launch_step(a, c->step_tl, c->step_to, c->n_wg, c->st);
    }
    if (coop_refusal(e)) {
        (void)hipGetLastError();
        c->coop_refused = true;
        c->step_state = 0;
        return kStepRefused;
    }
    if (e != hipSuccess) return fail(c, TF_HIP_EDEVICE, std::string("step kernel launch: ") + hipGetErrorString(e));
    c->epoch += (uint32_t)((uint64_t)n * (6ull * (uint64_t)p.n_layer + 8ull));
    return 0;
}

// Writes att_start and mode of the device control block.
int set_ctl(tf_hip_ctx* c, int att_start, int mode) {
    c->ctl_host->att_start = att_start;
    c->ctl_host->mode = mode;
    HIPCHK(c, hipMemcpyAsync((char*)c->ctl + offsetof(Ctl, att_start), (char*)c->ctl_host + offsetof(Ctl, att_start),
                             2 * sizeof(int32_t), hipMemcpyHostToDevice, c->st));
    return 0;
}

// n tokens on the context's decode path, from position c->pos: the step kernel when
// *use_step, else n replays of the captured graph. A refused cooperative launch switches
// the context to the graph path and runs the tokens there (*use_step then reads 0).
int run_tokens(tf_hip_ctx* c, int* use_step, int n, int greedy, int lm_every, int att_start) {
    if (*use_step) {
        const int rc = run_step(c, n, greedy, lm_every, att_start);
        if (rc != kStepRefused) return rc;
        *use_step = 0;
        const int g = ensure_graph(c);
        if (g) return g;
    }
    for (int i = 0; i < n; ++i) HIPCHK(c, hipGraphLaunch(c->gexec, c->st));
    return 0;
}

// Decides once, after every tensor is uploaded, whether prompts run on the matrix
// cores: every layer matrix in a format k_pf_gemm handles with row lengths it tiles,
// and a head size and GQA ratio k_pf_attn handles. Allocates the chunk buffers.
// Returns 1 (matrix cores), 0 (per-token path) or < 0.
int ensure_pf(tf_hip_ctx* c) {
    if (c->pf_opt != TF_HIP_PREFILL_MFMA) return 0;
    if (c->pf_state >= 0) return c->pf_state;
    int rc = check_ready(c);
    if (rc) return rc;
    c->pf_state = 0;
    const tf_hip_hparams& p = c->hp;
    for (int l = 0; l < p.n_layer; ++l) {
        auto M = [&](int k) -> const DevMat& { return mat(c, TF_HIP_SLOT_LAYER(l, k)); };
        const int kinds[7] = {TF_HIP_LAYER_Q,    TF_HIP_LAYER_K,  TF_HIP_LAYER_V,   TF_HIP_LAYER_O,
                              TF_HIP_LAYER_GATE, TF_HIP_LAYER_UP, TF_HIP_LAYER_DOWN};
        for (int k : kinds)
            if (!pf_gemm_supported(M(k).type, M(k).K, M(k).N)) return 0;
        // gate and up run in one launch, which takes one format
        if (M(TF_HIP_LAYER_GATE).type != M(TF_HIP_LAYER_UP).type) return 0;
    }
    if (!pf_attn_supported(p.head_dim, p.n_head / p.n_kv_head)) return 0;
    if (!c->px) {
        // rows of a chunk, padded to the large GEMM tiles' 128 (kPfChunk is a multiple)
        const int cap = std::min((p.max_seq + 127) / 128 * 128, kPfChunk);
        const size_t D = (size_t)p.n_embd, F = (size_t)p.n_ff, NQ = (size_t)c->H + 2 * (size_t)c->KVd;
        const size_t kmax = std::max({D, F, (size_t)c->H});
        if ((rc = dalloc(c, &c->px, cap * D * 4)) || (rc = dalloc(c, &c->pqkv, cap * NQ * 4)) ||
            (rc = dalloc(c, &c->patt, cap * (size_t)c->H * 4)) || (rc = dalloc(c, &c->ph, cap * F * 4)) ||
            (rc = dalloc(c, &c->prs, (size_t)cap * 4)) || (rc = dalloc(c, &c->pxa, cap * kmax * 2 * 2)))
            return rc;
        // up to 8 K slices of the widest non-SILU output (QKV or d_model)
        c->ppart_floats = 8 * (size_t)cap * std::max(NQ, D);
        if ((rc = dalloc(c, &c->ppart, c->ppart_floats * 4))) return rc;
        // attention of a chunk covers at most max_seq positions
        c->pattn_ws_bytes = pf_attn_ws_bytes(p.head_dim, p.n_kv_head, p.max_seq);
        if ((rc = dalloc(c, &c->pattn_ws, c->pattn_ws_bytes))) return rc;
        c->pf_cap = cap;
    }
    HIPCHK(c, hipStreamSynchronize(c->st));
    c->pf_state = 1;
    return 1;
}

// Rows [r0, r0 + n) of a layer matrix as a matrix of its own: its streams advanced by r0
// rows (the per-row strides of the DevMat layout of each format, as Fmt<T>::row reads them).
DevMat devmat_rows(const DevMat& m, int64_t r0, int64_t n) {
    DevMat d = m;
    int64_t q = 0, q2 = 0, sc = 0, s2 = 0;  // bytes per row of the q, q2, s and s2 streams
    switch (m.type) {
        case TF_HIP_TYPE_Q8_0: q = m.K; sc = m.K / 32 * 2; break;
        case TF_HIP_TYPE_Q4_0: q = m.K / 2; sc = m.K / 32 * 2; break;
        case TF_HIP_TYPE_Q4_1: q = m.K / 2; sc = m.K / 32 * 4; break;
        case TF_HIP_TYPE_Q6_K: q = m.K / 2; q2 = m.K / 4; sc = m.K / 16; s2 = m.K / 256 * 2; break;
        case TF_HIP_TYPE_F16: q = m.K * 2; break;
        default: q = m.K * 4; break;  // F32
    }
    d.q = m.q ? m.q + r0 * q : nullptr;
    d.q2 = m.q2 ? m.q2 + r0 * q2 : nullptr;
    d.s = m.s ? m.s + r0 * sc : nullptr;
    d.s2 = m.s2 ? m.s2 + r0 * s2 : nullptr;
    d.N = n;
    return d;
}

// n prompt tokens, staged at hist[c->pos ..], through the matrix-core layers in chunks
// of pf_cap rows; attention of every chunk covers the prompt from c->pos (the reference
// attends within the prefill call only, attention.cpp:82-111). Ends with the lm_head of
// the last row; the per-layer taps hold that row.
int prefill_mfma(tf_hip_ctx* c, int n) {
    const tf_hip_hparams& p = c->hp;
    const int D = p.n_embd, F = p.n_ff, Hd = c->H, KVd = c->KVd, NQ = Hd + 2 * KVd;
    const int start = c->pos;
    hipError_t e = hipSuccess;
    auto chk = [&](hipError_t r) {
        if (e == hipSuccess) e = r;
    };
    int nc = 0;
    for (int c0 = 0; c0 < n && e == hipSuccess; c0 += nc) {
        nc = std::min(c->pf_cap, n - c0);
        // beyond one 64-row tile, whole 128-row tiles: the large-tile GEMMs take any row count
        const int Mpad = nc <= kPfTileM ? kPfTileM : (nc + 127) / 128 * 128;
        const int pos0 = start + c0;
        const bool last = c0 + nc == n;
        chk(launch_embed_rows(mat(c, TF_HIP_SLOT_TOKEN_EMBD), c->hist + pos0, nc, c->px, D, c->st));
        auto base = [&](int K) {
            PfGemmArgs a;
            a.xa = c->pxa;
            a.rs = c->prs;
            a.part = c->ppart;
            a.part_floats = c->ppart_floats;
            a.K = K;
            a.M = nc;
            a.Mpad = Mpad;
            return a;
        };
        auto seg = [&](PfGemmArgs& a, int slot, float* y, int64_t ldy, const float* bias) {
            PfSeg& s = a.seg[a.n_seg++];
            const DevMat& w = mat(c, slot);
            s.w = w;
            s.y = y;
            s.ldy = ldy;
            s.bias = bias;
            s.sub0 = a.n_sub;
            a.n_sub += (int)(w.N / 16);
        };
        // the residual GEMMs' split-K reduce also splits their rows for the next GEMM when it
        // can (launch_pf_gemm says whether it did)
        auto fuse_split = [&](PfGemmArgs& a, const float* norm_w) {
            a.split_xa = c->pxa;
            a.split_rs = c->prs;
            a.split_w = norm_w;
            a.split_eps = p.rms_eps;
        };
        bool x_split = false;  // the attention-norm split of px is in pxa already
        for (int l = 0; l < p.n_layer && e == hipSuccess; ++l) {
            auto M = [&](int k) { return TF_HIP_SLOT_LAYER(l, k); };
            auto V = [&](int k) { return vec(c, TF_HIP_SLOT_LAYER(l, k)); };
            float* kc = c->kc + (size_t)l * c->kv_layer;
            float* vc = c->vc + (size_t)l * c->kv_layer;
            if (!x_split)
                chk(launch_pf_split(c->px, D, V(TF_HIP_LAYER_ATTN_NORM), p.rms_eps, D, nc, Mpad, c->pxa, c->prs,
                                    c->st));
            x_split = false;
            const int tq = mat(c, M(TF_HIP_LAYER_Q)).type;
            if (mat(c, M(TF_HIP_LAYER_K)).type != tq || mat(c, M(TF_HIP_LAYER_V)).type != tq) {
                // q, k and v in different formats: a launch each, then rope and the cache
                const int kinds[3] = {TF_HIP_LAYER_Q, TF_HIP_LAYER_K, TF_HIP_LAYER_V};
                const int bias[3] = {TF_HIP_LAYER_BQ, TF_HIP_LAYER_BK, TF_HIP_LAYER_BV};
                const int off[3] = {0, Hd, Hd + KVd};
                for (int i = 0; i < 3; ++i) {
                    PfGemmArgs a = base(D);
                    a.mode = GEMV_STORE;
                    seg(a, M(kinds[i]), c->pqkv + off[i], NQ, V(bias[i]));
                    chk(launch_pf_gemm(a, c->st));
                }
                chk(launch_pf_rope_store(c->pqkv, NQ, nc, p.n_head, p.n_kv_head, p.head_dim, c->rope_cos, c->rope_sin,
                                         pos0, kc, vc, p.kv_layout, p.max_seq, c->st));
            } else {
                PfGemmArgs a = base(D);
                a.mode = GEMV_STORE;
                seg(a, M(TF_HIP_LAYER_Q), c->pqkv, NQ, V(TF_HIP_LAYER_BQ));
                seg(a, M(TF_HIP_LAYER_K), c->pqkv + Hd, NQ, V(TF_HIP_LAYER_BK));
                seg(a, M(TF_HIP_LAYER_V), c->pqkv + Hd + KVd, NQ, V(TF_HIP_LAYER_BV));
                a.rope_cos = c->rope_cos;
                a.rope_sin = c->rope_sin;
                a.kc = kc;
                a.vc = vc;
                a.pos0 = pos0;
                a.n_head = p.n_head;
                a.n_kv = p.n_kv_head;
                a.hd = p.head_dim;
                a.kv_layout = p.kv_layout;
                a.max_seq = p.max_seq;
                bool done = false;
                chk(launch_pf_gemm(a, c->st, &done));
                if (!done)
                    chk(launch_pf_rope_store(c->pqkv, NQ, nc, p.n_head, p.n_kv_head, p.head_dim, c->rope_cos,
                                             c->rope_sin, pos0, kc, vc, p.kv_layout, p.max_seq, c->st));
            }
            chk(launch_pf_attn(c->pqkv, NQ, kc, vc, p.kv_layout, p.n_head, p.n_kv_head, p.head_dim, p.max_seq, nc,
                               pos0, start, c->patt, Hd, c->pattn_ws, c->pattn_ws_bytes, c->st));
            chk(launch_pf_split(c->patt, Hd, nullptr, 0.0f, Hd, nc, Mpad, c->pxa, c->prs, c->st));
            {
                PfGemmArgs a = base(Hd);
                a.mode = GEMV_RESID;
                seg(a, M(TF_HIP_LAYER_O), c->px, D, nullptr);
                fuse_split(a, V(TF_HIP_LAYER_FFN_NORM));
                bool done = false;
                chk(launch_pf_gemm(a, c->st, &done));
                if (!done)
                    chk(launch_pf_split(c->px, D, V(TF_HIP_LAYER_FFN_NORM), p.rms_eps, D, nc, Mpad, c->pxa,
                                        c->prs, c->st));
            }
            {
                // gate/up's large tiles (128 output columns) past whole rounds over the CUs: the
                // columns of the whole rounds in one launch, the rest in a second, which splits
                // its K to fill the CUs — when the rest is at most half a round (a 640-row chunk:
                // 255 + 65 tiles instead of two rounds; with more, its slices take a round too)
                const int cus = device_cu_count(), MT = Mpad % 128 == 0 ? Mpad / 128 : 0;
                const int ncol = F % 128 == 0 ? F / 128 : 0, n_big = ncol * MT;
                int ncA = ncol;
                if (n_big > cus && n_big % cus != 0) {
                    const int a_cols = n_big / cus * cus / MT;
                    if ((ncol - a_cols) * MT <= cus / 2) ncA = a_cols;
                }
                auto gateup = [&](int c0, int c1, bool fuse, bool* done) {
                    PfGemmArgs a = base(D);
                    a.mode = GEMV_SILU;
                    PfSeg& sg = a.seg[a.n_seg++];
                    sg.w = devmat_rows(mat(c, M(TF_HIP_LAYER_GATE)), c0, c1 - c0);
                    sg.w2 = devmat_rows(mat(c, M(TF_HIP_LAYER_UP)), c0, c1 - c0);
                    sg.y = c->ph + c0;
                    sg.ldy = F;
                    sg.bias = nullptr;
                    sg.sub0 = 0;
                    a.n_sub = (c1 - c0) / 16;
                    if (fuse) {  // a K-split reduce also splits the hidden rows
                        a.split_xa = c->pxa;
                        a.split_rs = c->prs;
                    }
                    chk(launch_pf_gemm(a, c->st, done));
                };
                bool done = false;
                if (ncA > 0 && ncA < ncol) {
                    gateup(0, ncA * 128, false, nullptr);
                    gateup(ncA * 128, F, false, nullptr);
                } else {
                    gateup(0, F, true, &done);
                }
                if (!done) chk(launch_pf_split(c->ph, F, nullptr, 0.0f, F, nc, Mpad, c->pxa, c->prs, c->st));
            }
            {
                PfGemmArgs a = base(F);
                a.mode = GEMV_RESID;
                seg(a, M(TF_HIP_LAYER_DOWN), c->px, D, nullptr);
                if (last) {
                    a.tap = c->taps + (size_t)l * D;
                    a.tap_row = nc - 1;
                }
                if (l + 1 < p.n_layer) fuse_split(a, vec(c, TF_HIP_SLOT_LAYER(l + 1, TF_HIP_LAYER_ATTN_NORM)));
                chk(launch_pf_gemm(a, c->st, &x_split));
            }
        }
    }
    chk(launch_pf_tail(c->ctl, start + n - 1, c->hist, c->px + (size_t)(nc - 1) * D, c->x, D, c->st));
    chk(launch_lm_head(c));
    if (e != hipSuccess) return fail(c, TF_HIP_EDEVICE, std::string("prefill launch: ") + hipGetErrorString(e));
    return 0;
}

int finish_step_outputs(tf_hip_ctx* c, float* logits, int32_t* argmax) {
    if (logits)
        HIPCHK(c, hipMemcpyAsync(logits, c->logits, (size_t)c->hp.n_vocab * 4, hipMemcpyDeviceToHost, c->st));
    HIPCHK(c, hipMemcpyAsync(c->ctl_host, c->ctl, sizeof(Ctl), hipMemcpyDeviceToHost, c->st));
    HIPCHK(c, hipStreamSynchronize(c->st));
    if (c->ctl_host->err == 2) return fail(c, TF_HIP_EDEVICE, "step kernel: an exchange wait timed out");
    if (c->ctl_host->err) return fail(c, TF_HIP_EDEVICE, "device reported an invalid token");
    if (c->ctl_host->pos != c->pos) return fail(c, TF_HIP_EDEVICE, "device position out of step");
    if (argmax) *argmax = key_to_index(c->ctl_host->key);
    return 0;
}

}  // namespace

extern "C" {

const char* tf_hip_last_error(const tf_hip_ctx* ctx) { return ctx ? ctx->err.c_str() : "null context"; }

int tf_hip_create(int device, const tf_hip_hparams* hp, tf_hip_ctx** out) {
    if (!hp || !out) return TF_HIP_EINVAL;
    *out = nullptr;
    const tf_hip_hparams& p = *hp;
    if (p.n_vocab <= 0 || p.n_embd <= 0 || p.n_ff <= 0 || p.n_layer <= 0 || p.n_head <= 0 || p.n_kv_head <= 0 ||
        p.max_seq <= 0)
        return TF_HIP_EINVAL;
    if (p.n_head % p.n_kv_head != 0 || p.n_head / p.n_kv_head > 8) return TF_HIP_EINVAL;
    if (p.head_dim != p.n_embd / p.n_head || p.head_dim % 8 != 0 || p.head_dim > 256) return TF_HIP_EINVAL;
    if (p.kv_layout != TF_HIP_KV_SEQ_MAJOR && p.kv_layout != TF_HIP_KV_HEAD_MAJOR) return TF_HIP_EINVAL;
    if (p.n_embd % 32 != 0 || p.n_ff % 32 != 0) return TF_HIP_EINVAL;

    tf_hip_ctx* c = new tf_hip_ctx();
    c->device = device;
    // TF_HIP_SPLIT_FROM: an override of the split-from span, read once here; ignored unless
    // it is a whole number in [0, 512]
    if (const char* sf = std::getenv("TF_HIP_SPLIT_FROM")) {
        char* end = nullptr;
        const long v = std::strtol(sf, &end, 10);
        if (end != sf && *end == 0 && v >= 0 && v <= kSplitFromMax) c->split_from = (int)v;
    }
    // TF_HIP_DECODE_PATH=step|graph: the initial decode path, for callers that do not
    // call tf_hip_set_decode_path (other values are ignored)
    if (const char* dp = std::getenv("TF_HIP_DECODE_PATH")) {
        const std::string v(dp);
        if (v == "step") c->path_opt = TF_HIP_PATH_STEP;
        if (v == "graph") c->path_opt = TF_HIP_PATH_GRAPH;
    }
    c->hp = p;
    c->H = p.n_head * p.head_dim;
    c->KVd = p.n_kv_head * p.head_dim;
    auto bail = [&](int rc) {
        tf_hip_destroy(c);
        return rc;
    };
    if (hipSetDevice(device) != hipSuccess) return bail(TF_HIP_EDEVICE);
    if (hipStreamCreateWithFlags(&c->st, hipStreamNonBlocking) != hipSuccess) return bail(TF_HIP_EDEVICE);
    const int n_slots = TF_HIP_SLOT_LAYER(p.n_layer, 0);
    c->mats.resize((size_t)n_slots);
    c->vecs.assign((size_t)n_slots, nullptr);
    c->vec_len.assign((size_t)n_slots, 0);

    const int S = attn_splits(p.max_seq);
    c->S = S;
    c->kv_layer = (size_t)p.n_kv_head * p.max_seq * p.head_dim;
    const size_t D = (size_t)p.n_embd;
    int rc = 0;
    if ((rc = dalloc(c, &c->kc, c->kv_layer * p.n_layer * 4)) || (rc = dalloc(c, &c->vc, c->kv_layer * p.n_layer * 4)) ||
        (rc = dalloc(c, &c->x, D * 4)) || (rc = dalloc(c, &c->q, (size_t)c->H * 4)) ||
        (rc = dalloc(c, &c->k, (size_t)c->KVd * 4)) || (rc = dalloc(c, &c->v, (size_t)c->KVd * 4)) ||
        (rc = dalloc(c, &c->att, (size_t)c->H * 4)) || (rc = dalloc(c, &c->h, (size_t)p.n_ff * 4)) ||
        (rc = dalloc(c, &c->logits, (size_t)p.n_vocab * 4)) ||
        (rc = dalloc(c, &c->taps, (size_t)(p.n_layer + 1) * D * 4)) ||
        (rc = dalloc(c, &c->part_o, (size_t)p.n_head * S * p.head_dim * 4)) ||
        (rc = dalloc(c, &c->part_ml, (size_t)p.n_head * S * 2 * 4)) ||
        (rc = dalloc(c, &c->ctl, sizeof(Ctl))) ||
        (rc = dalloc(c, &c->hist, (size_t)p.max_seq * 4)) ||
        (rc = dalloc(c, &c->rope_cos, (size_t)p.max_seq * (p.head_dim / 2) * 4)) ||
        (rc = dalloc(c, &c->rope_sin, (size_t)p.max_seq * (p.head_dim / 2) * 4)))
        return bail(rc);
    if (hipHostMalloc((void**)&c->ctl_host, sizeof(Ctl), 0) != hipSuccess) return bail(TF_HIP_ENOMEM);
    if (hipHostMalloc((void**)&c->tok_host, (size_t)p.max_seq * 4, 0) != hipSuccess) return bail(TF_HIP_ENOMEM);
    std::memset(c->ctl_host, 0, sizeof(Ctl));
    if (hipMemset(c->ctl, 0, sizeof(Ctl)) != hipSuccess || hipMemset(c->kc, 0, c->kv_layer * p.n_layer * 4) != hipSuccess ||
        hipMemset(c->vc, 0, c->kv_layer * p.n_layer * 4) != hipSuccess ||
        hipMemset(c->taps, 0, (size_t)(p.n_layer + 1) * D * 4) != hipSuccess)
        return bail(TF_HIP_EDEVICE);
    if (hipEventCreate(&c->ev0) != hipSuccess || hipEventCreate(&c->ev1) != hipSuccess) return bail(TF_HIP_EDEVICE);
    if (const char* lg = std::getenv("TF_HIP_LOG"); lg && *lg && std::strcmp(lg, "0") != 0)
        std::fprintf(stderr, "tf_hip: device %d kv=%s max_seq=%d layers=%d dim=%d heads=%d/%d\n", device,
                     p.kv_layout == TF_HIP_KV_HEAD_MAJOR ? "head" : "seq", p.max_seq, p.n_layer, p.n_embd,
                     p.n_head, p.n_kv_head);
    *out = c;
    return 0;
}

int tf_hip_destroy(tf_hip_ctx* c) {
    if (!c) return 0;
    (void)hipSetDevice(c->device);
    if (c->st) (void)hipStreamSynchronize(c->st);
    if (c->gexec) (void)hipGraphExecDestroy(c->gexec);
    if (c->graph) (void)hipGraphDestroy(c->graph);
    for (void* p : c->allocs) (void)hipFree(p);
    if (c->ctl_host) (void)hipHostFree(c->ctl_host);
    if (c->tok_host) (void)hipHostFree(c->tok_host);
    if (c->ev0) (void)hipEventDestroy(c->ev0);
    if (c->ev1) (void)hipEventDestroy(c->ev1);
    if (c->st) (void)hipStreamDestroy(c->st);
    delete c;
    return 0;
}

int tf_hip_upload_tensor(tf_hip_ctx* c, int slot, int t, int64_t ne0, int64_t ne1, const void* host, size_t nbytes) {
    if (!c) return TF_HIP_EINVAL;
    const tf_hip_hparams& p = c->hp;
    if (slot < 0 || slot >= (int)c->mats.size() || (slot > 2 && slot < 16) || !host)
        return fail(c, TF_HIP_EINVAL, "bad tensor slot " + std::to_string(slot));
    if (blck_elems(t) == 0) return fail(c, TF_HIP_EINVAL, "unsupported ggml type " + std::to_string(t));
    if (ne0 <= 0 || ne1 <= 0 || ne0 % blck_elems(t) != 0)
        return fail(c, TF_HIP_EINVAL, "row length not divisible by block size");
    if (nbytes != gguf_nbytes(t, ne0, ne1)) return fail(c, TF_HIP_EINVAL, "tensor byte size does not match its shape");
    if (c->gexec) {
        (void)hipGraphExecDestroy(c->gexec);
        (void)hipGraphDestroy(c->graph);
        c->gexec = nullptr;
        c->graph = nullptr;
    }
    HIPCHK(c, hipSetDevice(c->device));
    // vectors: norms and biases are read as raw F32 by the reference (model.cpp:87, layers.cpp:11)
    int kind = -1;
    if (slot >= 16) kind = (slot - 16) % TF_HIP_LAYER_COUNT;
    const bool is_vec = slot == TF_HIP_SLOT_OUTPUT_NORM || kind == TF_HIP_LAYER_ATTN_NORM ||
                        kind == TF_HIP_LAYER_FFN_NORM || kind == TF_HIP_LAYER_BQ || kind == TF_HIP_LAYER_BK ||
                        kind == TF_HIP_LAYER_BV;
    if (is_vec) {
        int64_t want = p.n_embd;
        if (kind == TF_HIP_LAYER_BQ) want = c->H;
        if (kind == TF_HIP_LAYER_BK || kind == TF_HIP_LAYER_BV) want = c->KVd;
        if (t != TF_HIP_TYPE_F32 || ne0 * ne1 != want)
            return fail(c, TF_HIP_EINVAL, "vector tensor must be F32 of length " + std::to_string(want));
        float* d = c->vecs[(size_t)slot];
        if (!d) {
            int rc = dalloc(c, &d, (size_t)want * 4);
            if (rc) return rc;
            c->vecs[(size_t)slot] = d;
            c->step_state = -1;
            c->pf_state = -1;
        }
        c->vec_len[(size_t)slot] = want;
        HIPCHK(c, hipMemcpy(d, host, (size_t)want * 4, hipMemcpyHostToDevice));
        return 0;
    }
    // matrices: expected [ne0 x ne1]
    int64_t K = 0, N = 0;
    if (slot == TF_HIP_SLOT_TOKEN_EMBD || slot == TF_HIP_SLOT_OUTPUT) {
        K = p.n_embd;
        N = p.n_vocab;
    } else {
        switch (kind) {
            case TF_HIP_LAYER_Q: K = p.n_embd; N = c->H; break;
            case TF_HIP_LAYER_K:
            case TF_HIP_LAYER_V: K = p.n_embd; N = c->KVd; break;
            case TF_HIP_LAYER_O: K = c->H; N = p.n_embd; break;
            case TF_HIP_LAYER_GATE:
            case TF_HIP_LAYER_UP: K = p.n_embd; N = p.n_ff; break;
            case TF_HIP_LAYER_DOWN: K = p.n_ff; N = p.n_embd; break;
        }
    }
    if (ne0 != K || ne1 != N)
        return fail(c, TF_HIP_EINVAL, "tensor shape [" + std::to_string(ne0) + " x " + std::to_string(ne1) +
                                           "] does not match the model, want [" + std::to_string(K) + " x " +
                                           std::to_string(N) + "]");
    if (!row_ok(t, K)) return fail(c, TF_HIP_EINVAL, "row length unsupported for this format");
    if (kind == TF_HIP_LAYER_UP || kind == TF_HIP_LAYER_GATE) {
        const int other = slot + (kind == TF_HIP_LAYER_UP ? -1 : 1);
        const DevMat& o = c->mats[(size_t)other];
        if (o.valid() && o.type != t) return fail(c, TF_HIP_EINVAL, "ffn_gate and ffn_up must share a format");
    }
    uint8_t* raw = nullptr;
    HIPCHK(c, hipMalloc(&raw, nbytes));
    hipError_t e = hipMemcpy(raw, host, nbytes, hipMemcpyHostToDevice);
    DevMat m;
    std::vector<void*> owned;
    if (e == hipSuccess) e = make_devmat(t, K, N, raw, m, owned, c->st);
    if (e == hipSuccess) e = hipStreamSynchronize(c->st);
    (void)hipFree(raw);
    if (e != hipSuccess) {
        for (void* q : owned) (void)hipFree(q);
        return fail(c, e == hipErrorOutOfMemory ? TF_HIP_ENOMEM : TF_HIP_EDEVICE,
                    std::string("upload: ") + hipGetErrorString(e));
    }
    c->allocs.insert(c->allocs.end(), owned.begin(), owned.end());
    c->mats[(size_t)slot] = m;  // a re-upload leaves the old streams allocated until destroy
    c->step_state = -1;         // the step kernel's layer table is rebuilt
    c->pf_state = -1;
    return 0;
}

int tf_hip_set_rope_table(tf_hip_ctx* c, const float* cos_tab, const float* sin_tab, int32_t n_pos, int32_t half) {
    if (!c || !cos_tab || !sin_tab) return TF_HIP_EINVAL;
    if (half != c->hp.head_dim / 2 || n_pos < c->hp.max_seq)
        return fail(c, TF_HIP_EINVAL, "RoPE table must be [>= max_seq][head_dim/2]");
    const size_t n = (size_t)c->hp.max_seq * half * 4;
    HIPCHK(c, hipSetDevice(c->device));
    HIPCHK(c, hipMemcpy(c->rope_cos, cos_tab, n, hipMemcpyHostToDevice));
    HIPCHK(c, hipMemcpy(c->rope_sin, sin_tab, n, hipMemcpyHostToDevice));
    c->rope_set = true;
    return 0;
}

int tf_hip_reset(tf_hip_ctx* c) {
    if (!c) return TF_HIP_EINVAL;
    HIPCHK(c, hipSetDevice(c->device));
    HIPCHK(c, hipStreamSynchronize(c->st));
    c->pos = 0;
    c->have_logits = false;
    std::memset(c->ctl_host, 0, sizeof(Ctl));
    c->ctl_host->epoch = c->epoch;  // exchange words keep old epochs: never reuse one
    HIPCHK(c, hipMemcpyAsync(c->ctl, c->ctl_host, sizeof(Ctl), hipMemcpyHostToDevice, c->st));
    HIPCHK(c, hipMemsetAsync(c->kc, 0, c->kv_layer * c->hp.n_layer * 4, c->st));
    HIPCHK(c, hipMemsetAsync(c->vc, 0, c->kv_layer * c->hp.n_layer * 4, c->st));
    HIPCHK(c, hipStreamSynchronize(c->st));
    return 0;
}

int tf_hip_get_pos(const tf_hip_ctx* c) { return c ? c->pos : TF_HIP_EINVAL; }

int tf_hip_decode(tf_hip_ctx* c, int32_t token, float* logits, int32_t* argmax) {
    if (!c) return TF_HIP_EINVAL;
    HIPCHK(c, hipSetDevice(c->device));
    if (c->pos >= c->hp.max_seq) return fail(c, TF_HIP_ERANGE, "decode exceeds max_seq");
    if (token < 0 || token >= mat(c, TF_HIP_SLOT_TOKEN_EMBD).N)
        return fail(c, TF_HIP_ERANGE, "token " + std::to_string(token) + " out of range");
    int use_step = ensure_step(c);
    if (use_step < 0) return use_step;
    int rc = use_step ? 0 : ensure_graph(c);
    if (rc) return rc;
    c->tok_host[0] = token;
    HIPCHK(c, hipMemcpyAsync(c->hist + c->pos, c->tok_host, 4, hipMemcpyHostToDevice, c->st));
    if ((rc = set_ctl(c, 0, 0))) return rc;
    if ((rc = run_tokens(c, &use_step, 1, 0, 1, 0))) return rc;
    c->pos += 1;
    rc = finish_step_outputs(c, logits, argmax);
    if (rc) return rc;
    c->have_logits = true;
    return 0;
}

int tf_hip_prefill(tf_hip_ctx* c, const int32_t* tokens, int32_t n, float* logits, int32_t* argmax) {
    if (!c || (n > 0 && !tokens)) return TF_HIP_EINVAL;
    if (n <= 0) return 0;
    HIPCHK(c, hipSetDevice(c->device));
    if (n > c->hp.max_seq - c->pos) return fail(c, TF_HIP_ERANGE, "prefill exceeds max_seq");
    const int64_t V = mat(c, TF_HIP_SLOT_TOKEN_EMBD).N;
    for (int i = 0; i < n; ++i)
        if (tokens[i] < 0 || tokens[i] >= V)
            return fail(c, TF_HIP_ERANGE, "token " + std::to_string(tokens[i]) + " out of range");
    const int use_pf = n >= 2 ? ensure_pf(c) : 0;
    if (use_pf < 0) return use_pf;
    int use_step = use_pf ? 0 : ensure_step(c);
    if (use_step < 0) return use_step;
    int rc = (use_pf || use_step) ? 0 : ensure_graph(c);
    if (rc) return rc;
    std::memcpy(c->tok_host, tokens, (size_t)n * 4);
    HIPCHK(c, hipMemcpyAsync(c->hist + c->pos, c->tok_host, (size_t)n * 4, hipMemcpyHostToDevice, c->st));
    if ((rc = set_ctl(c, c->pos, 0))) return rc;
    HIPCHK(c, hipEventRecord(c->ev0, c->st));
    if (use_pf) {
        if ((rc = prefill_mfma(c, n))) return rc;
    } else if ((rc = run_tokens(c, &use_step, n, 0, 0, c->pos))) {
        return rc;
    }
    HIPCHK(c, hipEventRecord(c->ev1, c->st));
    c->pos += n;
    rc = finish_step_outputs(c, logits, argmax);
    if (rc) return rc;
    HIPCHK(c, hipEventElapsedTime(&c->last_ms, c->ev0, c->ev1));
    c->last_steps = use_pf ? 1 : (use_step ? 1 : n);
    c->last_name = use_pf ? "prefill_mfma" : (use_step ? "k_step" : "decode_graph");
    c->have_logits = true;
    return 0;
}

int tf_hip_generate(tf_hip_ctx* c, int32_t n, int32_t* out) {
    if (!c || (n > 0 && !out)) return TF_HIP_EINVAL;
    if (n <= 0) return 0;
    HIPCHK(c, hipSetDevice(c->device));
    if (!c->have_logits) return fail(c, TF_HIP_ESTATE, "generate needs a prior prefill or decode");
    if (n > c->hp.max_seq - c->pos) return fail(c, TF_HIP_ERANGE, "decode exceeds max_seq");
    int use_step = ensure_step(c);
    if (use_step < 0) return use_step;
    int rc = use_step ? 0 : ensure_graph(c);
    if (rc) return rc;
    const int pos0 = c->pos;
    if ((rc = set_ctl(c, 0, 1))) return rc;
    HIPCHK(c, hipEventRecord(c->ev0, c->st));
    if ((rc = run_tokens(c, &use_step, n, 1, 1, 0))) return rc;
    HIPCHK(c, hipEventRecord(c->ev1, c->st));
    HIPCHK(c, hipMemcpyAsync(c->tok_host, c->hist + pos0, (size_t)n * 4, hipMemcpyDeviceToHost, c->st));
    c->pos += n;
    rc = finish_step_outputs(c, nullptr, nullptr);
    if (rc) return rc;
    std::memcpy(out, c->tok_host, (size_t)n * 4);
    HIPCHK(c, hipEventElapsedTime(&c->last_ms, c->ev0, c->ev1));
    c->last_steps = use_step ? 1 : n;
    c->last_name = use_step ? "k_step" : "decode_graph";
    return 0;
}

int tf_hip_set_decode_path(tf_hip_ctx* c, int32_t path) {
    if (!c || (path != TF_HIP_PATH_GRAPH && path != TF_HIP_PATH_STEP))
        return TF_HIP_EINVAL;
    c->path_opt = path;
    if (path != TF_HIP_PATH_GRAPH && c->step_state == 0) c->step_state = -1;  // decide again
    return 0;
}

int tf_hip_get_hparams(const tf_hip_ctx* c, tf_hip_hparams* out) {
    if (!c || !out) return TF_HIP_EINVAL;
    *out = c->hp;
    return 0;
}

int tf_hip_test_refuse_cooperative(tf_hip_ctx* c, int32_t n) {
    if (!c || n < 0) return TF_HIP_EINVAL;
    c->refuse_coop = n;
    return 0;
}

int tf_hip_set_split_all_from(tf_hip_ctx* c, int32_t span) {
    if (!c) return TF_HIP_EINVAL;
    c->split_all_from = span < 0 ? -1 : span;
    return 0;
}

int tf_hip_set_split_from(tf_hip_ctx* c, int32_t span) {
    if (!c) return TF_HIP_EINVAL;
    if (span < 0) {
        c->split_from = kSplitFromDefault;
        return 0;
    }
    if (span > kSplitFromMax)
        return fail(c, TF_HIP_EINVAL, "split_from " + std::to_string(span) + " above " + std::to_string(kSplitFromMax));
    c->split_from = span;
    return 0;
}

int tf_hip_get_step_config(tf_hip_ctx* c, int32_t* out, int32_t n) {
    if (!c || !out || n < 5) return TF_HIP_EINVAL;
    HIPCHK(c, hipSetDevice(c->device));
    const int s = ensure_step(c);
    if (s < 0) return s;
    if (s == 0) return fail(c, TF_HIP_ESTATE, "the step kernel does not run this model");
    const tf_hip_hparams& p = c->hp;
    out[0] = c->n_wg;
    out[1] = c->step_split;
    out[2] = c->step_split_all;
    out[3] = c->split_from;
    out[4] = c->split_all_from >= 0 ? c->split_all_from
                                    : step_split_all_from(p.n_head, p.n_kv_head, p.head_dim, c->step_split);
    return 0;
}

int tf_hip_set_exchange_epoch(tf_hip_ctx* c, uint32_t epoch) {
    if (!c) return TF_HIP_EINVAL;
    HIPCHK(c, hipSetDevice(c->device));
    HIPCHK(c, hipStreamSynchronize(c->st));
    c->epoch = epoch;
    c->ctl_host->epoch = epoch;
    HIPCHK(c, hipMemcpy((char*)c->ctl + offsetof(Ctl, epoch), (char*)c->ctl_host + offsetof(Ctl, epoch),
                        sizeof(uint32_t), hipMemcpyHostToDevice));
    return 0;
}

int tf_hip_set_prefill_path(tf_hip_ctx* c, int32_t path) {
    if (!c || (path != TF_HIP_PREFILL_TOKENS && path != TF_HIP_PREFILL_MFMA)) return TF_HIP_EINVAL;
    c->pf_opt = path;
    if (path == TF_HIP_PREFILL_MFMA && c->pf_state == 0) c->pf_state = -1;
    return 0;
}

int tf_hip_get_prefill_path(tf_hip_ctx* c) {
    if (!c) return TF_HIP_EINVAL;
    HIPCHK(c, hipSetDevice(c->device));
    const int s = ensure_pf(c);
    return s < 0 ? s : (s ? TF_HIP_PREFILL_MFMA : TF_HIP_PREFILL_TOKENS);
}

int tf_hip_get_decode_path(tf_hip_ctx* c) {
    if (!c) return TF_HIP_EINVAL;
    HIPCHK(c, hipSetDevice(c->device));
    const int s = ensure_step(c);
    return s < 0 ? s : (s ? TF_HIP_PATH_STEP : TF_HIP_PATH_GRAPH);
}

int tf_hip_get_layer_act(tf_hip_ctx* c, int32_t layer, float* out) {
    if (!c || !out || layer < 0 || layer > c->hp.n_layer) return TF_HIP_EINVAL;
    HIPCHK(c, hipSetDevice(c->device));
    HIPCHK(c, hipStreamSynchronize(c->st));
    HIPCHK(c, hipMemcpy(out, c->taps + (size_t)layer * c->hp.n_embd, (size_t)c->hp.n_embd * 4, hipMemcpyDeviceToHost));
    return 0;
}

int tf_hip_read_kv(tf_hip_ctx* c, int32_t layer, int32_t which, int32_t pos0, int32_t n, float* out) {
    if (!c || !out || layer < 0 || layer >= c->hp.n_layer || pos0 < 0 || n < 0 || pos0 > c->hp.max_seq ||
        n > c->hp.max_seq - pos0)
        return TF_HIP_EINVAL;
    HIPCHK(c, hipSetDevice(c->device));
    HIPCHK(c, hipStreamSynchronize(c->st));
    const tf_hip_hparams& p = c->hp;
    const float* base = (which ? c->vc : c->kc) + (size_t)layer * c->kv_layer;
    const size_t hd = (size_t)p.head_dim;
    if (p.kv_layout == TF_HIP_KV_SEQ_MAJOR) {
        HIPCHK(c, hipMemcpy(out, base + (size_t)pos0 * p.n_kv_head * hd, (size_t)n * p.n_kv_head * hd * 4,
                            hipMemcpyDeviceToHost));
    } else {
        for (int g = 0; g < p.n_kv_head; ++g)
            HIPCHK(c, hipMemcpy2D(out + g * hd, (size_t)p.n_kv_head * hd * 4, base + ((size_t)g * p.max_seq + pos0) * hd,
                                  hd * 4, hd * 4, (size_t)n, hipMemcpyDeviceToHost));
    }
    return 0;
}

int tf_hip_last_timing(const tf_hip_ctx* c, float* total_ms, float* kernel_ms, int32_t* launches, char* name,
                       int32_t name_len) {
    if (!c) return TF_HIP_EINVAL;
    if (total_ms) *total_ms = c->last_ms;
    if (kernel_ms) *kernel_ms = c->last_ms;
    if (launches) *launches = c->last_steps;
    if (name && name_len > 0) std::snprintf(name, (size_t)name_len, "%s", c->last_name);
    return 0;
}

// Profiling variant of tf_hip_generate: the same kernels launched one by one with
// events around each, per kernel class: summed ms, launches and algorithmic bytes.
int tf_hip_profile_generate(tf_hip_ctx* c, int32_t n, int32_t* out, float* ms_by_class, int32_t* launches_by_class,
                            double* bytes_by_class) {
    if (!c || n <= 0 || !out) return TF_HIP_EINVAL;
    HIPCHK(c, hipSetDevice(c->device));
    if (!c->have_logits) return fail(c, TF_HIP_ESTATE, "generate needs a prior prefill or decode");
    if (n > c->hp.max_seq - c->pos) return fail(c, TF_HIP_ERANGE, "decode exceeds max_seq");
    int rc = check_ready(c);
    if (rc) return rc;
    const int pos0 = c->pos;
    if ((rc = set_ctl(c, 0, 1))) return rc;
    Prof prof;
    for (int i = 0; i < n; ++i) {
        const hipError_t e = enqueue_step(c, &prof, pos0 + i, 0);
        if (e != hipSuccess) return fail(c, TF_HIP_EDEVICE, std::string("profile step: ") + hipGetErrorString(e));
    }
    HIPCHK(c, hipMemcpyAsync(c->tok_host, c->hist + pos0, (size_t)n * 4, hipMemcpyDeviceToHost, c->st));
    c->pos += n;
    rc = finish_step_outputs(c, nullptr, nullptr);
    if (rc) return rc;
    std::memcpy(out, c->tok_host, (size_t)n * 4);
    for (int k = 0; k < kNumClasses; ++k) {
        if (ms_by_class) ms_by_class[k] = 0;
        if (launches_by_class) launches_by_class[k] = 0;
        if (bytes_by_class) bytes_by_class[k] = 0;
    }
    for (size_t i = 0; i < prof.cls.size(); ++i) {
        float ms = 0;
        (void)hipEventElapsedTime(&ms, prof.ev[2 * i], prof.ev[2 * i + 1]);
        const int k = prof.cls[i];
        if (ms_by_class) ms_by_class[k] += ms;
        if (launches_by_class) launches_by_class[k] += 1;
        if (bytes_by_class) bytes_by_class[k] += prof.bytes[i];
    }
    for (hipEvent_t e : prof.ev) (void)hipEventDestroy(e);
    return 0;
}

const char* tf_hip_kernel_class_name(int32_t k) { return (k >= 0 && k < kNumClasses) ? kClassNames[k] : ""; }

}  // extern "C"

// ---------------------------------------------------------------- op-level entry points

namespace {

struct OpScope {
    hipStream_t st = nullptr;
    std::vector<void*> mem;
    ~OpScope() {
        if (st) (void)hipStreamSynchronize(st);
        for (void* p : mem) (void)hipFree(p);
        if (st) (void)hipStreamDestroy(st);
    }
    template <typename T>
    hipError_t alloc(T** p, size_t bytes) {
        void* d = nullptr;
        hipError_t e = hipMalloc(&d, bytes ? bytes : 16);
        if (e == hipSuccess) mem.push_back(d);
        *p = (T*)d;
        return e;
    }
};

#define OPCHK(call)                                                                   \
    do {                                                                              \
        hipError_t e_ = (call);                                                       \
        if (e_ != hipSuccess) return e_ == hipErrorOutOfMemory ? TF_HIP_ENOMEM : TF_HIP_EDEVICE; \
    } while (0)

int op_begin(int device, OpScope& s) {
    OPCHK(hipSetDevice(device));
    OPCHK(hipStreamCreateWithFlags(&s.st, hipStreamNonBlocking));
    return 0;
}

int op_upload_mat(OpScope& s, int t, const void* w, int64_t K, int64_t N, DevMat& m) {
    uint8_t* raw = nullptr;
    const size_t nb = gguf_nbytes(t, K, N);
    OPCHK(s.alloc(&raw, nb));
    OPCHK(hipMemcpy(raw, w, nb, hipMemcpyHostToDevice));
    OPCHK(make_devmat(t, K, N, raw, m, s.mem, s.st));
    return 0;
}

}  // namespace

extern "C" {

int tf_hip_dequant_rows(int device, int t, const void* w, int64_t ne0, int64_t ne1, int64_t row0, int64_t nrows,
                        float* out) {
    if (!w || !out || blck_elems(t) == 0 || !row_ok(t, ne0) || ne1 <= 0 || row0 < 0 || nrows <= 0 ||
        row0 + nrows > ne1)
        return TF_HIP_EINVAL;
    OpScope s;
    int rc = op_begin(device, s);
    if (rc) return rc;
    DevMat m;
    const size_t rb = gguf_nbytes(t, ne0, 1);
    if ((rc = op_upload_mat(s, t, (const uint8_t*)w + row0 * rb, ne0, nrows, m))) return rc;
    float* d_out = nullptr;
    OPCHK(s.alloc(&d_out, (size_t)nrows * ne0 * 4));
    OPCHK(launch_dequant_rows(m, 0, nrows, d_out, s.st));
    OPCHK(hipMemcpyAsync(out, d_out, (size_t)nrows * ne0 * 4, hipMemcpyDeviceToHost, s.st));
    OPCHK(hipStreamSynchronize(s.st));
    return 0;
}

int tf_hip_matmul(int device, int t, const void* w, int64_t ne0, int64_t ne1, const float* x, int32_t n_rows_x,
                  float* y) {
    if (!w || !x || !y || blck_elems(t) == 0 || !row_ok(t, ne0) || ne1 <= 0 || n_rows_x <= 0) return TF_HIP_EINVAL;
    OpScope s;
    int rc = op_begin(device, s);
    if (rc) return rc;
    DevMat m;
    if ((rc = op_upload_mat(s, t, w, ne0, ne1, m))) return rc;
    float *dx = nullptr, *dy = nullptr;
    OPCHK(s.alloc(&dx, (size_t)n_rows_x * ne0 * 4));
    OPCHK(s.alloc(&dy, (size_t)n_rows_x * ne1 * 4));
    OPCHK(hipMemcpy(dx, x, (size_t)n_rows_x * ne0 * 4, hipMemcpyHostToDevice));
    if (n_rows_x >= 2 && pf_gemm_supported(t, ne0, ne1)) {
        // several rows: the prefill GEMM on the matrix cores
        const int Mpad = (n_rows_x + kPfTileM - 1) / kPfTileM * kPfTileM;
        uint16_t* xa;
        float* rs;
        OPCHK(s.alloc(&xa, (size_t)Mpad * ne0 * 2 * 2));
        OPCHK(s.alloc(&rs, (size_t)Mpad * 4));
        OPCHK(launch_pf_split(dx, ne0, nullptr, 0.0f, (int)ne0, n_rows_x, Mpad, xa, rs, s.st));
        PfGemmArgs a;
        a.xa = xa;
        a.rs = rs;
        // workspace for K slices (up to 8 of them, as a model context's chunk buffers hold)
        a.part_floats = (size_t)8 * Mpad * ne1;
        OPCHK(s.alloc(&a.part, a.part_floats * 4));
        a.K = (int)ne0;
        a.M = n_rows_x;
        a.Mpad = Mpad;
        a.mode = GEMV_STORE;
        a.n_seg = 1;
        a.seg[0].w = m;
        a.seg[0].y = dy;
        a.seg[0].ldy = ne1;
        a.n_sub = (int)(ne1 / 16);
        OPCHK(launch_pf_gemm(a, s.st));
        OPCHK(hipMemcpyAsync(y, dy, (size_t)n_rows_x * ne1 * 4, hipMemcpyDeviceToHost, s.st));
        OPCHK(hipStreamSynchronize(s.st));
        return 0;
    }
    const int R = pick_rows(ne1);
    for (int i = 0; i < n_rows_x; ++i) {
        GemvArgs a;
        a.type = t;
        a.K = ne0;
        a.mode = GEMV_STORE;
        a.x = dx + (size_t)i * ne0;
        add_seg(a, m, dy + (size_t)i * ne1, nullptr, nullptr, R);
        OPCHK(launch_gemv(a, R, s.st));
    }
    OPCHK(hipMemcpyAsync(y, dy, (size_t)n_rows_x * ne1 * 4, hipMemcpyDeviceToHost, s.st));
    OPCHK(hipStreamSynchronize(s.st));
    return 0;
}

int tf_hip_rmsnorm(int device, const float* x, const float* w, int32_t n, int32_t rows, float eps, float* out) {
    if (!x || !w || !out || n <= 0 || rows <= 0) return TF_HIP_EINVAL;
    OpScope s;
    int rc = op_begin(device, s);
    if (rc) return rc;
    float *dx, *dw, *dout;
    OPCHK(s.alloc(&dx, (size_t)n * rows * 4));
    OPCHK(s.alloc(&dw, (size_t)n * 4));
    OPCHK(s.alloc(&dout, (size_t)n * rows * 4));
    OPCHK(hipMemcpy(dx, x, (size_t)n * rows * 4, hipMemcpyHostToDevice));
    OPCHK(hipMemcpy(dw, w, (size_t)n * 4, hipMemcpyHostToDevice));
    OPCHK(launch_rmsnorm_rows(dx, dw, n, rows, eps, dout, s.st));
    OPCHK(hipMemcpyAsync(out, dout, (size_t)n * rows * 4, hipMemcpyDeviceToHost, s.st));
    OPCHK(hipStreamSynchronize(s.st));
    return 0;
}

int tf_hip_rope(int device, float* x, int32_t seq, int32_t n_heads, int32_t hd, int32_t pos0, const float* cos_tab,
                const float* sin_tab, int32_t n_pos_tab) {
    if (!x || !cos_tab || !sin_tab || seq <= 0 || n_heads <= 0 || hd <= 0 || hd % 2 || pos0 < 0 || n_pos_tab <= 0 ||
        seq > n_pos_tab - pos0)
        return TF_HIP_EINVAL;
    OpScope s;
    int rc = op_begin(device, s);
    if (rc) return rc;
    const size_t nx = (size_t)seq * n_heads * hd, nt = (size_t)(pos0 + seq) * (hd / 2);
    float *dx, *dc, *ds;
    OPCHK(s.alloc(&dx, nx * 4));
    OPCHK(s.alloc(&dc, nt * 4));
    OPCHK(s.alloc(&ds, nt * 4));
    OPCHK(hipMemcpy(dx, x, nx * 4, hipMemcpyHostToDevice));
    OPCHK(hipMemcpy(dc, cos_tab, nt * 4, hipMemcpyHostToDevice));
    OPCHK(hipMemcpy(ds, sin_tab, nt * 4, hipMemcpyHostToDevice));
    OPCHK(launch_rope_rows(dx, seq, n_heads, hd, pos0, dc, ds, s.st));
    OPCHK(hipMemcpyAsync(x, dx, nx * 4, hipMemcpyDeviceToHost, s.st));
    OPCHK(hipStreamSynchronize(s.st));
    return 0;
}

int tf_hip_attn_prefill(int device, const float* q, const float* k, const float* v, int32_t seq, int32_t n_heads,
                        int32_t n_kv, int32_t hd, float* out) {
    if (!q || !k || !v || !out || seq <= 0 || n_heads <= 0 || n_kv <= 0 || n_heads % n_kv ||
        !pf_attn_supported(hd, n_heads / n_kv))
        return TF_HIP_EINVAL;
    OpScope s;
    int rc = op_begin(device, s);
    if (rc) return rc;
    const size_t nq = (size_t)seq * n_heads * hd, nk = (size_t)seq * n_kv * hd;
    float *dq, *dk, *dv, *dout;
    OPCHK(s.alloc(&dq, nq * 4));
    OPCHK(s.alloc(&dk, nk * 4));
    OPCHK(s.alloc(&dv, nk * 4));
    OPCHK(s.alloc(&dout, nq * 4));
    OPCHK(hipMemcpy(dq, q, nq * 4, hipMemcpyHostToDevice));
    OPCHK(hipMemcpy(dk, k, nk * 4, hipMemcpyHostToDevice));
    OPCHK(hipMemcpy(dv, v, nk * 4, hipMemcpyHostToDevice));
    // k and v rows [seq][n_kv][hd] are a sequence-major cache of seq positions
    const size_t ws_bytes = pf_attn_ws_bytes(hd, n_kv, seq);
    void* ws = nullptr;
    OPCHK(s.alloc(&ws, ws_bytes));
    OPCHK(launch_pf_attn(dq, (int64_t)n_heads * hd, dk, dv, TF_HIP_KV_SEQ_MAJOR, n_heads, n_kv, hd, seq, seq, 0, 0,
                         dout, (int64_t)n_heads * hd, ws, ws_bytes, s.st));
    OPCHK(hipMemcpyAsync(out, dout, nq * 4, hipMemcpyDeviceToHost, s.st));
    OPCHK(hipStreamSynchronize(s.st));
    return 0;
}

int tf_hip_attn_decode(int device, const float* q, const float* k_rows, const float* v_rows, int32_t n_heads,
                       int32_t n_kv, int32_t hd, int32_t n_pos, int32_t max_seq, int32_t layout, float* out) {
    if (!q || !k_rows || !v_rows || !out || n_heads <= 0 || n_kv <= 0 || n_heads % n_kv || n_heads / n_kv > 8 ||
        hd % 8 || hd > 256 || hd <= 0 || n_pos <= 0 || n_pos > max_seq || (layout != 0 && layout != 1))
        return TF_HIP_EINVAL;
    OpScope s;
    int rc = op_begin(device, s);
    if (rc) return rc;
    const size_t cache = (size_t)n_kv * max_seq * hd;
    std::vector<float> hk(cache, 0.0f), hv(cache, 0.0f);
    for (int p = 0; p < n_pos; ++p)
        for (int g = 0; g < n_kv; ++g) {
            const size_t o = layout ? ((size_t)g * max_seq + p) * hd : ((size_t)p * n_kv + g) * hd;
            std::memcpy(&hk[o], k_rows + ((size_t)p * n_kv + g) * hd, (size_t)hd * 4);
            std::memcpy(&hv[o], v_rows + ((size_t)p * n_kv + g) * hd, (size_t)hd * 4);
        }
    const int S = attn_splits(max_seq);
    float *dq, *dk, *dv, *dout, *pk, *pv, *po, *pml;
    OPCHK(s.alloc(&dq, (size_t)n_heads * hd * 4));
    OPCHK(s.alloc(&dk, cache * 4));
    OPCHK(s.alloc(&dv, cache * 4));
    OPCHK(s.alloc(&dout, (size_t)n_heads * hd * 4));
    OPCHK(s.alloc(&pk, (size_t)n_kv * hd * 4));
    OPCHK(s.alloc(&pv, (size_t)n_kv * hd * 4));
    OPCHK(s.alloc(&po, (size_t)n_heads * S * hd * 4));
    OPCHK(s.alloc(&pml, (size_t)n_heads * S * 2 * 4));
    OPCHK(hipMemcpy(dq, q, (size_t)n_heads * hd * 4, hipMemcpyHostToDevice));
    OPCHK(hipMemcpy(dk, hk.data(), cache * 4, hipMemcpyHostToDevice));
    OPCHK(hipMemcpy(dv, hv.data(), cache * 4, hipMemcpyHostToDevice));
    OPCHK(hipMemcpy(pk, k_rows + (size_t)(n_pos - 1) * n_kv * hd, (size_t)n_kv * hd * 4, hipMemcpyHostToDevice));
    OPCHK(hipMemcpy(pv, v_rows + (size_t)(n_pos - 1) * n_kv * hd, (size_t)n_kv * hd * 4, hipMemcpyHostToDevice));
    AttnArgs a{};
    a.q = dq;
    a.knew = pk;
    a.vnew = pv;
    a.kc = dk;
    a.vc = dv;
    a.rope_cos = dq;  // unused with rope = 0
    a.rope_sin = dq;
    a.part_o = po;
    a.part_ml = pml;
    a.out = dout;
    a.ctl = nullptr;
    a.H = n_heads;
    a.G = n_kv;
    a.hd = hd;
    a.max_seq = max_seq;
    a.layout = layout;
    a.S = S;
    a.rope = 0;
    a.store_kv = 0;
    a.fixed_pos = n_pos - 1;
    a.fixed_start = 0;
    OPCHK(launch_attn_decode(a, s.st));
    OPCHK(hipMemcpyAsync(out, dout, (size_t)n_heads * hd * 4, hipMemcpyDeviceToHost, s.st));
    OPCHK(hipStreamSynchronize(s.st));
    return 0;
}

}  // extern "C"

// ---------------------------------------------------------------- allocation-free attention

namespace {

// Device scratch of tf_hip_attn_decode_noalloc: the split partials (o, then m and l) of
// one call. Each GPU the library runs on holds its own copy until the process ends.
constexpr size_t kScratchFloats = TF_HIP_ATTN_SCRATCH_BYTES / sizeof(float);
static __device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on `device` (the current device), looked up once per
// device. In host code the array's name is only a stand-in; kernels get this address. The
// lookup may load the library's code objects, which a stream under graph capture must not
// see: while `st` is capturing, a device whose address is not known yet gets TF_HIP_ESTATE
// before anything is enqueued (its first call has to be made outside capture).
int scratch_on(int device, hipStream_t st, float** out) {
    if (device < 0 || device >= kMaxDevices) return TF_HIP_EINVAL;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(st, &cs) != hipSuccess) return TF_HIP_EDEVICE;
        if (cs != hipStreamCaptureStatusNone) return TF_HIP_ESTATE;
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return TF_HIP_EDEVICE;
        g_scratch_ptr[device] = (float*)p;
    }
    *out = g_scratch_ptr[device];
    return 0;
}

}  // namespace

extern "C" {

int tf_hip_attn_decode_noalloc(int device, const float* q, const float* k_cache, const float* v_cache,
                               int32_t n_heads, int32_t n_kv, int32_t hd, int32_t n_pos, int32_t max_seq,
                               int32_t layout, float* out, void* stream) {
    if (!q || !k_cache || !v_cache || !out || n_heads <= 0 || n_kv <= 0 || n_heads % n_kv || n_heads / n_kv > 8 ||
        hd % 8 || hd > 256 || hd <= 0 || n_pos <= 0 || n_pos > max_seq || (layout != 0 && layout != 1))
        return TF_HIP_EINVAL;
    const int S = attn_splits(max_seq);
    // o partials [n_heads][S][hd], then (m, l) pairs [n_heads][S][2]
    const size_t need = (size_t)n_heads * S * hd + (size_t)n_heads * S * 2;
    if (S > 1 && need > kScratchFloats) return TF_HIP_ESCRATCH;
    if (hipSetDevice(device) != hipSuccess) return TF_HIP_EDEVICE;
    float* ptr = nullptr;
    int rc = scratch_on(device, (hipStream_t)stream, &ptr);
    if (rc) return rc;
    AttnArgs a{};
    a.q = q;
    a.knew = nullptr;  // the row at n_pos - 1 is read from the cache
    a.vnew = nullptr;
    a.kc = const_cast<float*>(k_cache);  // read only: store_kv = 0
    a.vc = const_cast<float*>(v_cache);
    a.rope_cos = q;  // unused: rope = 0
    a.rope_sin = q;
    a.part_o = ptr;
    a.part_ml = ptr + (size_t)n_heads * S * hd;
    a.out = out;
    a.ctl = nullptr;
    a.H = n_heads;
    a.G = n_kv;
    a.hd = hd;
    a.max_seq = max_seq;
    a.layout = layout;
    a.S = S;
    a.rope = 0;
    a.store_kv = 0;
    a.fixed_pos = n_pos - 1;
    a.fixed_start = 0;
    return launch_attn_decode(a, (hipStream_t)stream) == hipSuccess ? 0 : TF_HIP_EDEVICE;
}

int tf_hip_sample(tf_hip_ctx* c, float temperature, float top_p, float r, int32_t* token) {
    if (!c || !token || !(r >= 0.0f && r < 1.0f) || top_p != top_p || temperature != temperature)
        return TF_HIP_EINVAL;
    if (!c->have_logits) return fail(c, TF_HIP_ESTATE, "sample needs a prior prefill, decode or generate");
    HIPCHK(c, hipSetDevice(c->device));
    const int V = c->hp.n_vocab;
    int rc;
    if (!c->d_sampled) {
        const size_t bytes = sample_work_bytes(V);
        if ((rc = dalloc(c, (uint8_t**)&c->sample_work, bytes)) || (rc = dalloc(c, &c->d_sampled, 64)) ||
            (rc = dalloc(c, &c->sample_ctl, sizeof(Ctl))))
            return rc;
        c->sample_bytes = bytes;
    }
    int32_t tok = 0;
    if (temperature <= 0.0f) {
        // sample_greedy (sampler.cpp:8-13), as sample_logits does for temperature <= 0
        HIPCHK(c, hipMemsetAsync(c->sample_ctl, 0, sizeof(Ctl), c->st));
        HIPCHK(c, launch_argmax(c->logits, V, c->sample_ctl, c->st));
        Ctl h;
        HIPCHK(c, hipMemcpyAsync(&h, c->sample_ctl, sizeof(Ctl), hipMemcpyDeviceToHost, c->st));
        HIPCHK(c, hipStreamSynchronize(c->st));
        tok = key_to_index(h.key);
    } else {
        HIPCHK(c, launch_sample(c->logits, V, temperature, top_p, r, c->sample_work, c->sample_bytes, c->d_sampled,
                                nullptr, nullptr, c->st));
        HIPCHK(c, hipMemcpyAsync(c->tok_host, c->d_sampled, 4, hipMemcpyDeviceToHost, c->st));
        HIPCHK(c, hipStreamSynchronize(c->st));
        tok = c->tok_host[0];
    }
    *token = tok;
    return 0;
}

int tf_hip_sample_logits(int device, const float* logits, int32_t n, float temperature, float top_p, float r,
                         int32_t* token, int32_t* sorted_idx, float* probs) {
    if (!logits || !token || n <= 0 || !(r >= 0.0f && r < 1.0f) || top_p != top_p || temperature != temperature)
        return TF_HIP_EINVAL;
    if (temperature <= 0.0f) return tf_hip_argmax(device, logits, n, token);
    OpScope s;
    int rc = op_begin(device, s);
    if (rc) return rc;
    float *dl, *dp = nullptr;
    int32_t *dt, *di = nullptr;
    void* work;
    const size_t bytes = sample_work_bytes(n);
    OPCHK(s.alloc(&dl, (size_t)n * 4));
    OPCHK(s.alloc(&dt, 64));
    OPCHK(s.alloc((uint8_t**)&work, bytes));
    if (sorted_idx) OPCHK(s.alloc(&di, (size_t)n * 4));
    if (probs) OPCHK(s.alloc(&dp, (size_t)n * 4));
    OPCHK(hipMemcpy(dl, logits, (size_t)n * 4, hipMemcpyHostToDevice));
    OPCHK(launch_sample(dl, n, temperature, top_p, r, work, bytes, dt, di, dp, s.st));
    OPCHK(hipMemcpyAsync(token, dt, 4, hipMemcpyDeviceToHost, s.st));
    if (sorted_idx) OPCHK(hipMemcpyAsync(sorted_idx, di, (size_t)n * 4, hipMemcpyDeviceToHost, s.st));
    if (probs) OPCHK(hipMemcpyAsync(probs, dp, (size_t)n * 4, hipMemcpyDeviceToHost, s.st));
    OPCHK(hipStreamSynchronize(s.st));
    return 0;
}

int tf_hip_argmax(int device, const float* x, int32_t n, int32_t* out) {
    if (!x || !out || n <= 0) return TF_HIP_EINVAL;
    OpScope s;
    int rc = op_begin(device, s);
    if (rc) return rc;
    float* dx;
    Ctl* ctl;
    OPCHK(s.alloc(&dx, (size_t)n * 4));
    OPCHK(s.alloc(&ctl, sizeof(Ctl)));
    OPCHK(hipMemcpy(dx, x, (size_t)n * 4, hipMemcpyHostToDevice));
    OPCHK(hipMemset(ctl, 0, sizeof(Ctl)));
    OPCHK(launch_argmax(dx, n, ctl, s.st));
    Ctl h;
    OPCHK(hipMemcpyAsync(&h, ctl, sizeof(Ctl), hipMemcpyDeviceToHost, s.st));
    OPCHK(hipStreamSynchronize(s.st));
    *out = key_to_index(h.key);
    return 0;
}

// The sum (mod 2^32) of the wave partials k_read_stream wrote to sink.
static uint32_t sink_total(const uint32_t* d_sink, size_t n, hipStream_t st, hipError_t* err) {
    std::vector<uint32_t> h(n);
    *err = hipMemcpyAsync(h.data(), d_sink, n * 4, hipMemcpyDeviceToHost, st);
    if (*err == hipSuccess) *err = hipStreamSynchronize(st);
    uint32_t t = 0;
    for (uint32_t v : h) t += v;
    return t;
}

int tf_hip_read_stream(int device, size_t nbytes, int32_t iters, double* best, double* median, uint32_t* checksum) {
    if (nbytes < 16 || iters <= 0 || !best || !median) return TF_HIP_EINVAL;
    OpScope s;
    int rc = op_begin(device, s);
    if (rc) return rc;
    const size_t n4 = nbytes / 16;
    uint4* p;
    uint32_t* sink;
    const int blocks = 8 * device_cu_count();
    const size_t n_sink = (size_t)blocks * kWavesPerBlock;
    OPCHK(s.alloc(&p, n4 * 16));
    OPCHK(s.alloc(&sink, n_sink * sizeof(uint32_t)));
    OPCHK(launch_fill_stream(p, n4, blocks, s.st));
    hipEvent_t e0, e1;
    OPCHK(hipEventCreate(&e0));
    OPCHK(hipEventCreate(&e1));
    std::vector<double> gbs;
    OPCHK(launch_read_stream(p, n4, sink, blocks, s.st));  // warm-up
    for (int i = 0; i < iters; ++i) {
        OPCHK(hipEventRecord(e0, s.st));
        OPCHK(launch_read_stream(p, n4, sink, blocks, s.st));
        OPCHK(hipEventRecord(e1, s.st));
        OPCHK(hipEventSynchronize(e1));
        float ms = 0;
        OPCHK(hipEventElapsedTime(&ms, e0, e1));
        gbs.push_back((double)n4 * 16 / (ms * 1e-3) / 1e9);
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    hipError_t e = hipSuccess;
    const uint32_t sum = sink_total(sink, n_sink, s.st, &e);
    OPCHK(e);
    if (checksum) *checksum = sum;
    std::sort(gbs.begin(), gbs.end());
    *best = gbs.back();
    *median = gbs[gbs.size() / 2];
    return 0;
}

int tf_hip_copy_stream(int device, size_t nbytes, int32_t iters, double* best, double* median, uint32_t* checksum) {
    if (nbytes < 16 || iters <= 0 || !best || !median) return TF_HIP_EINVAL;
    OpScope s;
    int rc = op_begin(device, s);
    if (rc) return rc;
    const size_t n4 = nbytes / 16;
    uint4 *src, *dst;
    uint32_t* sink;
    const int blocks = 8 * device_cu_count();
    const size_t n_sink = (size_t)blocks * kWavesPerBlock;
    OPCHK(s.alloc(&src, n4 * 16));
    OPCHK(s.alloc(&dst, n4 * 16));
    OPCHK(s.alloc(&sink, n_sink * sizeof(uint32_t)));
    OPCHK(launch_fill_stream(src, n4, blocks, s.st));
    OPCHK(hipMemsetAsync(dst, 0, n4 * 16, s.st));
    hipEvent_t e0, e1;
    OPCHK(hipEventCreate(&e0));
    OPCHK(hipEventCreate(&e1));
    std::vector<double> gbs;
    OPCHK(launch_copy_stream(dst, src, n4, blocks, s.st));  // warm-up
    for (int i = 0; i < iters; ++i) {
        OPCHK(hipEventRecord(e0, s.st));
        OPCHK(launch_copy_stream(dst, src, n4, blocks, s.st));
        OPCHK(hipEventRecord(e1, s.st));
        OPCHK(hipEventSynchronize(e1));
        float ms = 0;
        OPCHK(hipEventElapsedTime(&ms, e0, e1));
        gbs.push_back(2.0 * (double)n4 * 16 / (ms * 1e-3) / 1e9);
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    // the copy's destination summed by the read stream's kernel
    OPCHK(launch_read_stream(dst, n4, sink, blocks, s.st));
    hipError_t e = hipSuccess;
    const uint32_t sum = sink_total(sink, n_sink, s.st, &e);
    OPCHK(e);
    if (checksum) *checksum = sum;
    std::sort(gbs.begin(), gbs.end());
    *best = gbs.back();
    *median = gbs[gbs.size() / 2];
    return 0;
}

}  // extern "C"
