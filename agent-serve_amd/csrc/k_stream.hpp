// Streaming persistent decode step for Q8_0 models: the token loop of k_step.hpp
// (Model::decode, model.cpp:197-208, and the per-token layers of Model::prefill,
// model.cpp:144-195) with the same phases, exchange protocol and per-element arithmetic,
// and the weights delivered by a wave of their own.
//
// A workgroup is 10 waves on one CU: 8 compute waves and 2 loader waves. The weights are
// repacked once (k_stream_pack) into one contiguous byte stream per (workgroup, compute
// wave): the slots that wave will consume in one token, in order -- its share of every
// layer's QKV, wo, gate/up and down rows, then of the lm_head. The loader waves copy the 8
// streams of their workgroup (4 each) into 8 LDS rings with direct global->LDS loads, two
// rounds of at most two slots per stream in flight, and keep doing so whatever the compute
// waves are waiting for: the
// compute waves never issue a weight load, so their exchange polls never queue behind
// one (a wave's loads complete in issue order), while HBM keeps streaming through the
// hand-offs. The compute waves synchronise among themselves with an LDS counter (the
// loaders take part in no barrier).
//
// A slot is one tile of a row: up to 64 lane steps of 16 weights. In the stream: q bytes
// (16 per step) then the fp16 block scales (1 byte per step), padded to 16 bytes. In LDS:
// 1024 q bytes then 64 scale bytes.
//
// Ring protocol, per compute wave w: ready[w] counts the slots whose loads have completed
// (a loader writes it after s_waitcnt vmcnt), released[w] the slots wave w has read
// (written after its reads complete). The loader fills a slot only while fewer than RS are
// unreleased; wave w reads slot k once ready[w] > k.
#pragma once
#include "k_step.hpp"

namespace tfk {

constexpr int kSCW = 8;                        // compute waves per workgroup
constexpr int kSLW = 2;                        // loader waves per workgroup
constexpr int kSThreads = (kSCW + kSLW) * kWave;
constexpr int kSlotBytes = 1088;               // LDS bytes per ring slot
constexpr int kSlotQ = 1024;                   // q bytes of a full slot (64 steps x 16)

// One phase of the stream: n_rows rows of K weights; T tiles (slots) per row, the last of
// `tail` lane steps; spu slots per unit (2 for gate/up: the gate tile and the up tile).
struct SPhase {
    int n_rows, K, T, tail, spu;
};

__host__ __device__ inline int split_lo(int n, int i, int parts) { return (int)((int64_t)n * i / parts); }

__host__ __device__ inline SPhase s_phase(int n_rows, int K, int spu) {
    SPhase p;
    p.n_rows = n_rows;
    p.K = K;
    const int steps = K / 16;
    p.T = (steps + 63) / 64;
    p.tail = steps - 64 * (p.T - 1);
    p.spu = spu;
    return p;
}

// Rows [r0, r0 + rows) of workgroup c; its units (row, tile) u0..u1 of compute wave w.
struct SUnits {
    int r0, rows, u0, u1;
};
__host__ __device__ inline SUnits s_units(const SPhase& p, int c, int nwg, int w) {
    SUnits u;
    u.r0 = split_lo(p.n_rows, c, nwg);
    u.rows = split_lo(p.n_rows, c + 1, nwg) - u.r0;
    const int U = u.rows * p.T;
    u.u0 = split_lo(U, w, kSCW);
    u.u1 = split_lo(U, w + 1, kSCW);
    return u;
}
__host__ __device__ inline int s_steps(const SPhase& p, int j) { return j == p.T - 1 ? p.tail : 64; }
__host__ __device__ inline int s_gbytes(int steps) { return steps * 16 + (steps + 15) / 16 * 16; }

// The five phases of the model (the same for every layer), in stream order.
enum { SP_QKV = 0, SP_WO = 1, SP_GU = 2, SP_DOWN = 3, SP_LM = 4, SP_COUNT = 5 };
struct SPlan {
    SPhase ph[SP_COUNT];
};
__host__ __device__ inline SPlan s_plan(int D, int F, int H, int G, int hd, int V) {
    SPlan s;
    s.ph[SP_QKV] = s_phase(H * hd + 2 * G * hd, D, 1);
    s.ph[SP_WO] = s_phase(D, H * hd, 1);
    s.ph[SP_GU] = s_phase(F, D, 2);
    s.ph[SP_DOWN] = s_phase(D, F, 1);
    s.ph[SP_LM] = s_phase(V, D, 1);
    return s;
}

// Per-layer inputs of the stream kernel besides the streamed matrices.
struct SLayer {
    const float* attn_norm;
    const float* ffn_norm;
    const float* bq;
    const float* bk;
    const float* bv;
    float* kc;
    float* vc;
};

struct StreamArgs {
    const SLayer* layers;
    const uint8_t* stream;      // the repacked weights
    const uint64_t* sbase;      // [nwg * 8] byte offset of each (workgroup, wave) stream
    const uint8_t* ssteps;      // lane steps of every slot of a token's stream, streams end to end
    const uint32_t* sfirst;     // [nwg * 8] first slot of each stream in ssteps
    const uint32_t* snl;        // [nwg * 8] slots of the layers' part of a token's stream
    const uint32_t* snt;        // [nwg * 8] slots of a whole token's stream (layers + lm_head)
    DevMat embd;                // token embedding (Q8_0)
    const float* out_norm;
    const float* rope_cos;
    const float* rope_sin;
    unsigned long long* ex;
    Ctl* ctl;
    int32_t* hist;
    float* logits;
    float* taps;
    int n_layer, D, F, H, G, hd, V, max_seq, layout;
    float eps;
    int n_tokens, greedy, lm_every, att_start;
    int split_all;              // splits per kv head of long spans (every workgroup splits), 0: none
    int split_from;             // spans up to this attend on one workgroup per kv head
    int ring_slots;             // RS: slots per compute wave's ring
    int steps_max;              // slots of the largest per-wave token stream (LDS steps table)
    unsigned long long* dbg;    // builds with TF_STREAM_PROBE: [nwg][64] cycle counts, or nullptr
};

}  // namespace tfk
