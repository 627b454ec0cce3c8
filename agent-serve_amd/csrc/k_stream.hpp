// Streaming persistent decode step for Q8_0 models: the token loop of k_step.hpp
// (Model::decode, model.cpp:197-208, and the per-token layers of Model::prefill,
// model.cpp:144-195) with the same phases, exchange protocol and per-element arithmetic,
// and the weights fed through LDS at a bounded depth.
//
// The weights are repacked once (k_stream_pack) into one contiguous byte stream per
// (workgroup, wave): the slots that wave will consume in one token, in order -- its share
// of every layer's QKV, wo, gate/up and down rows, then of the lm_head. Each wave copies its
// own stream into an LDS ring of its own with direct global->LDS loads and keeps at most a
// few slots in flight: the CU's vector memory path is one queue, and an exchange poll
// waits behind every load the CU has in flight (one-way hand-offs measured on MI355X: 0.57
// us idle, 1.3 us at 16 KiB in flight per CU, 2.4 us at 32 KiB and more), while 16 KiB per
// CU already streams 5.9 of the 6.3 TB/s the chip reads. The ring is topped up after every
// slot a wave consumes and on every round of an exchange poll, so HBM keeps streaming
// through the hand-offs at that depth.
//
// A slot is one tile of a row: up to 64 lane steps of 16 weights. In the stream: q bytes
// (16 per step) then the fp16 block scales (1 byte per step), padded to 16 bytes. In LDS:
// 1024 q bytes then 64 scale bytes. Every slot is two load instructions (q, scales), so a
// wave knows slot k is in LDS once at most 2 j of its loads are outstanding, j being the
// slots it issued after k (its loads complete in order).
#pragma once
#include "k_step.hpp"

namespace tfk {

constexpr int kSCW = 8;                        // waves per workgroup
constexpr int kSThreads = kSCW * kWave;
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
    int ring_slots;             // RS: slots per wave's ring
    int steps_max;              // slots of the largest per-wave token stream (LDS steps table)
    int depth;                  // slots a wave keeps in flight in the layer phases
    int depth_lm;               // and in the lm_head phase (no hand-off waits behind its loads)
    unsigned long long* dbg;    // builds with TF_STREAM_PROBE: [nwg][64] time stamps, or nullptr
};

}  // namespace tfk
