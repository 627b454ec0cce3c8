// Temperature / nucleus sampling of one logits vector on the GPU: sample_logits
// (sampler.cpp:15-52) with the reference's arithmetic, so that the same uniform draw picks
// the same token.
//
//   1. the indices sorted by descending logit (an LSD radix sort of 8-bit digits, stable:
//      equal logits keep ascending indices; std::sort leaves their order unspecified);
//   2. p_i = exp((l_i - max) / T) for every i, with the reference libm's expf (expf_libm.hpp);
//   3. s = p_0 + p_1 + ... in that order, p_i /= s;
//   4. nucleus (top_p < 1): the running sum until it reaches top_p gives the kept count
//      `last` and z (the same sum, so the same float), p_i /= z for i < last;
//   5. the first i whose running sum reaches the draw r, else the last kept index.
//
// Steps 2 and the divisions run on every thread; the running sums (3-5) are sequential
// float additions in the reference, so one wave performs them in order from registers
// (64 values per load, eight loads ahead), one lane-broadcast addition per element. A sum
// stops early once the next value is at most a quarter of an ulp of the sum: the values
// do not increase, so none of the rest can change it (sharp distributions stop after a
// handful of elements; a nearly flat one over a 128K vocabulary takes the whole pass).
#include "dev_common.hpp"
#include "expf_libm.hpp"
#include "tf_internal.hpp"

namespace tfk {
namespace {

constexpr int kSampleThreads = 1024;

// expf_libm's table in constant memory
__constant__ uint64_t kExp2Tab[32] = TF_EXP2_TABLE;

// ---- radix sort of (key, index) pairs
// Keys: the logits mapped to unsigned integers whose ascending order is the logits'
// descending order (-0 taken as +0, as `>` compares them equal). Each wave owns a tile
// of kRsTile consecutive elements; a pass counts the tile's digits, an exclusive scan over
// [digit][tile] turns the counts into offsets, and the wave scatters its tile in index
// order (lanes of a 64-element step that share a digit are ranked by lane), so the sort
// is stable.
constexpr int kRsTile = 1024;
constexpr int kRsWaves = kBlock / kWave;

__device__ __forceinline__ uint32_t desc_key(float f) {
    uint32_t u = __float_as_uint(f == 0.0f ? 0.0f : f);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);  // ascending float order
    return ~u;
}

__global__ __launch_bounds__(kBlock) void k_rs_init(const float* logits, uint32_t* key, int32_t* val, int n) {
    for (int i = blockIdx.x * kBlock + threadIdx.x; i < n; i += gridDim.x * kBlock) {
        key[i] = desc_key(logits[i]);
        val[i] = i;
    }
}

__global__ __launch_bounds__(kBlock) void k_rs_hist(const uint32_t* key, int n, int shift, uint32_t* hist,
                                                    int tiles) {
    __shared__ uint32_t cnt[kRsWaves][256];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int tile = blockIdx.x * kRsWaves + wv;
    for (int d = lane; d < 256; d += kWave) cnt[wv][d] = 0;
    __syncthreads();
    if (tile < tiles) {
        const int end = min(n, (tile + 1) * kRsTile);
        for (int i = tile * kRsTile + lane; i < end; i += kWave) atomicAdd(&cnt[wv][(key[i] >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tile < tiles)
        for (int d = lane; d < 256; d += kWave) hist[(size_t)d * tiles + tile] = cnt[wv][d];
}

// Exclusive prefix sum of m counts in place (one workgroup).
__global__ __launch_bounds__(1024) void k_rs_scan(uint32_t* hist, int m) {
    __shared__ uint32_t part[1024];
    const int t = threadIdx.x;
    const int per = (m + 1023) / 1024;
    const int b = t * per, e = min(m, b + per);
    uint32_t sum = 0;
    for (int i = b; i < e; ++i) sum += hist[i];
    part[t] = sum;
    __syncthreads();
    for (int o = 1; o < 1024; o <<= 1) {
        const uint32_t v = t >= o ? part[t - o] : 0u;
        __syncthreads();
        part[t] += v;
        __syncthreads();
    }
    uint32_t run = part[t] - sum;
    for (int i = b; i < e; ++i) {
        const uint32_t c = hist[i];
        hist[i] = run;
        run += c;
    }
}

__global__ __launch_bounds__(kBlock) void k_rs_scatter(const uint32_t* kin, const int32_t* vin, uint32_t* kout,
                                                       int32_t* vout, int n, int shift, const uint32_t* hist,
                                                       int tiles) {
    __shared__ uint32_t off[kRsWaves][256];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int tile = blockIdx.x * kRsWaves + wv;
    if (tile >= tiles) return;  // whole waves: no barrier below
    for (int d = lane; d < 256; d += kWave) off[wv][d] = hist[(size_t)d * tiles + tile];
    const uint64_t below = (1ull << lane) - 1ull;
    const int end = min(n, (tile + 1) * kRsTile);
    for (int i0 = tile * kRsTile; i0 < end; i0 += kWave) {
        const int i = i0 + lane;
        const bool valid = i < end;
        const uint32_t k = valid ? kin[i] : 0u;
        const uint32_t d = (k >> shift) & 255u;
        uint64_t peers = __ballot(valid);
#pragma unroll
        for (int bit = 0; bit < 8; ++bit) {
            const uint64_t set = __ballot((d >> bit) & 1u);
            peers &= ((d >> bit) & 1u) ? set : ~set;
        }
        const uint32_t base = valid ? off[wv][d] : 0u;
        if (valid) {
            const uint32_t dst = base + (uint32_t)__popcll(peers & below);
            kout[dst] = k;
            vout[dst] = vin[i];
            if ((peers >> lane) == 1ull) off[wv][d] = base + (uint32_t)__popcll(peers);  // the group's last lane
        }
    }
}

// The next float above s minus s (s >= 0 finite), a quarter of it: values at or below
// this cannot change s when added.
__device__ __forceinline__ float quarter_ulp(float s) {
    return (__uint_as_float(__float_as_uint(s) + 1u) - s) * 0.25f;
}

// Wave 0's view of p[0..n): 64 values per register, eight registers per refill, the next
// eight loading while these are consumed.
struct Seq {
    const float* p;
    int n, lane;
    float cur[8], nxt[8];
    __device__ void load(int base, float (&b)[8]) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const int i = base + 64 * c + lane;
            b[c] = i < n ? p[i] : 0.0f;
        }
    }
};

// Steps 2-5 for the logits in the order idx (one workgroup).
__global__ __launch_bounds__(kSampleThreads) void k_sample(const float* logits, const int32_t* idx, float* p, int n,
                                                           float temperature, float top_p, float r, int32_t* out) {
    __shared__ float sh_s, sh_z;
    __shared__ int sh_last;
    const int tid = threadIdx.x, lane = tid & 63;
    const bool w0 = tid < 64;
    const float m = logits[idx[0]];
    for (int i = tid; i < n; i += kSampleThreads) p[i] = expf_libm((logits[idx[i]] - m) / temperature, kExp2Tab);
    __syncthreads();
    Seq q{p, n, lane};
    // 3: s in order
    if (w0) {
        float s = 0.0f;
        q.load(0, q.cur);
        for (int base = 0; base < n; base += 512) {
            q.load(base + 512, q.nxt);
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const int cb = base + 64 * c;
                if (cb < n) {
                    if (__int_as_float(__builtin_amdgcn_readlane(__float_as_int(q.cur[c]), 0)) <= quarter_ulp(s))
                        goto s_done;
                    const int cnt = min(64, n - cb);
                    for (int j = 0; j < cnt; ++j) s += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(q.cur[c]), j));
                }
            }
#pragma unroll
            for (int c = 0; c < 8; ++c) q.cur[c] = q.nxt[c];
        }
    s_done:
        if (lane == 0) sh_s = s;
    }
    __syncthreads();
    const float s = sh_s;
    for (int i = tid; i < n; i += kSampleThreads) p[i] = p[i] / s;
    __syncthreads();
    // 4: nucleus
    if (w0) {
        int last = n;
        float acc = 0.0f;
        if (top_p < 1.0f) {
            q.load(0, q.cur);
            for (int base = 0; base < n; base += 512) {
                q.load(base + 512, q.nxt);
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    const int cb = base + 64 * c;
                    if (cb < n) {
                        // stuck below top_p: the sum never reaches it, every value stays
                        if (__int_as_float(__builtin_amdgcn_readlane(__float_as_int(q.cur[c]), 0)) <= quarter_ulp(acc))
                            goto p_done;
                        const int cnt = min(64, n - cb);
                        for (int j = 0; j < cnt; ++j) {
                            acc += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(q.cur[c]), j));
                            if (acc >= top_p) {
                                last = cb + j + 1;
                                goto p_done;
                            }
                        }
                    }
                }
#pragma unroll
                for (int c = 0; c < 8; ++c) q.cur[c] = q.nxt[c];
            }
        }
    p_done:
        if (lane == 0) {
            sh_last = last;
            sh_z = acc;
        }
    }
    __syncthreads();
    const int last = sh_last;
    if (top_p < 1.0f) {
        const float z = sh_z;
        for (int i = tid; i < last; i += kSampleThreads) p[i] = p[i] / z;
        __syncthreads();
    }
    // 5: the draw
    if (w0) {
        int tok = idx[last - 1];
        float acc = 0.0f;
        Seq f{p, last, lane};
        f.load(0, f.cur);
        for (int base = 0; base < last; base += 512) {
            f.load(base + 512, f.nxt);
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const int cb = base + 64 * c;
                if (cb < last) {
                    // stuck below r: no later element is picked
                    if (__int_as_float(__builtin_amdgcn_readlane(__float_as_int(f.cur[c]), 0)) <= quarter_ulp(acc))
                        goto r_done;
                    const int cnt = min(64, last - cb);
                    for (int j = 0; j < cnt; ++j) {
                        acc += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f.cur[c]), j));
                        if (r <= acc) {
                            tok = idx[cb + j];
                            goto r_done;
                        }
                    }
                }
            }
#pragma unroll
            for (int c = 0; c < 8; ++c) f.cur[c] = f.nxt[c];
        }
    r_done:
        if (lane == 0) *out = tok;
    }
}

}  // namespace

size_t sample_work_bytes(int n) {
    const size_t a = ((size_t)n * 4 + 255) / 256 * 256;
    const size_t tiles = ((size_t)n + kRsTile - 1) / kRsTile;
    return 5 * a + (256 * tiles * 4 + 255) / 256 * 256;
}

hipError_t launch_sample(const float* logits, int n, float temperature, float top_p, float r, void* work,
                         size_t work_bytes, int32_t* d_token, int32_t* d_sorted_idx, float* d_probs, hipStream_t st) {
    const size_t a = ((size_t)n * 4 + 255) / 256 * 256;
    if (work_bytes < sample_work_bytes(n)) return hipErrorInvalidValue;
    uint8_t* w = (uint8_t*)work;
    uint32_t* key[2] = {(uint32_t*)w, (uint32_t*)(w + a)};
    int32_t* val[2] = {(int32_t*)(w + 2 * a), (int32_t*)(w + 3 * a)};
    float* p = d_probs ? d_probs : (float*)(w + 4 * a);
    uint32_t* hist = (uint32_t*)(w + 5 * a);
    const int tiles = (n + kRsTile - 1) / kRsTile;
    const int blocks = (tiles + kRsWaves - 1) / kRsWaves;
    hipLaunchKernelGGL(k_rs_init, dim3((n + kBlock - 1) / kBlock), dim3(kBlock), 0, st, logits, key[0], val[0], n);
    for (int pass = 0; pass < 4; ++pass) {
        const int src = pass & 1;
        hipLaunchKernelGGL(k_rs_hist, dim3(blocks), dim3(kBlock), 0, st, key[src], n, 8 * pass, hist, tiles);
        hipLaunchKernelGGL(k_rs_scan, dim3(1), dim3(1024), 0, st, hist, 256 * tiles);
        hipLaunchKernelGGL(k_rs_scatter, dim3(blocks), dim3(kBlock), 0, st, key[src], val[src], key[src ^ 1],
                           val[src ^ 1], n, 8 * pass, hist, tiles);
    }
    // four passes: the sorted indices are back in val[0]
    const int32_t* idx = val[0];
    if (d_sorted_idx) {
        hipError_t e = hipMemcpyAsync(d_sorted_idx, idx, (size_t)n * 4, hipMemcpyDeviceToDevice, st);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(k_sample, dim3(1), dim3(kSampleThreads), 0, st, logits, idx, p, n, temperature, top_p, r,
                       d_token);
    return hipGetLastError();
}

}  // namespace tfk
