// Per-format lane steps over the HBM layout of DevMat.
//
// A step is one aligned 16-byte load of the primary stream plus its scales:
//   Q8_0 16 elements, Q4_0/Q4_1/Q6_K 32 elements, F16 8, F32 4.
// load() fetches a step of one row; dot() returns its contribution to x . w with x
// (and its 16-element partial sums x16) in LDS; dequant() writes the step's values.
//
// Q8_0 bytes stay signed: each converts with one v_cvt_f32_i32 (SDWA byte select with
// sign extension), so the dot is sum_j x_j q_j directly and its rounding scales with
// sum |x_j q_j|. The 4- and 6-bit formats decode unsigned codes u = q + c with one
// v_cvt_f32_ubyte each, and sum_j x_j q_j = sum_j x_j u_j - c * sum_j x_j, where the
// per-16 sums of x come from the prologue. dequant() produces d * (float)q exactly as
// the reference does (quant.cpp:66-131: all those products are exact).
#pragma once

#include "dev_common.hpp"
#include "tf_internal.hpp"

namespace tfk {

struct RowPtr {
    const uint8_t* q;
    const uint8_t* q2;
    const uint8_t* s;
    const uint8_t* s2;
};

template <int T>
struct Fmt;

// ---------------------------------------------------------------- Q8_0
template <>
struct Fmt<TF_HIP_TYPE_Q8_0> {
    static constexpr int E = 16;
    static constexpr bool kNeedSums = false;
    struct Raw {
        uint4 q;
        uint32_t d;
    };
    __device__ static RowPtr row(const DevMat& m, int64_t r) {
        return {m.q + r * m.K, nullptr, m.s + r * (m.K / 32) * 2, nullptr};
    }
    __device__ static Raw load(const RowPtr& p, int s) {
        Raw w;
        w.q = gload_u4(p.q + 16 * (int64_t)s);
        w.d = *gptr((const uint16_t*)(p.s + 2 * (s >> 1)));
        return w;
    }
    // sum_j x_j q_j of the step's 16 elements, then times d (dot_q8_0_f32 scales each
    // block's sum by d, quant.cpp:266-321)
    __device__ static float dot(const Raw& w, const float* xs, const float*, int s) {
        const float4* x4 = (const float4*)(xs + 16 * s);
        float t = 0.0f;
        const uint32_t q[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 xv = x4[i];
            t = fmaf(xv.x, sb0(q[i]), t);
            t = fmaf(xv.y, sb1(q[i]), t);
            t = fmaf(xv.z, sb2(q[i]), t);
            t = fmaf(xv.w, sb3(q[i]), t);
        }
        return h2f(w.d) * t;
    }
    // dot() with the step's 16 inputs already loaded (the same operations in the same order)
    __device__ static float dot_x(const Raw& w, const float4 (&x)[4]) {
        float t = 0.0f;
        const uint32_t q[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            t = fmaf(x[i].x, sb0(q[i]), t);
            t = fmaf(x[i].y, sb1(q[i]), t);
            t = fmaf(x[i].z, sb2(q[i]), t);
            t = fmaf(x[i].w, sb3(q[i]), t);
        }
        return h2f(w.d) * t;
    }
    __device__ static void dequant(const Raw& w, float* out) {
        const float d = h2f(w.d);
        const uint32_t q[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
#pragma unroll
        for (int i = 0; i < 16; ++i) out[i] = d * (float)(int8_t)(q[i >> 2] >> (8 * (i & 3)));
    }
};

// ---------------------------------------------------------------- Q4_0
template <>
struct Fmt<TF_HIP_TYPE_Q4_0> {
    static constexpr int E = 32;
    static constexpr bool kNeedSums = true;
    struct Raw {
        uint4 q;
        uint32_t d;
    };
    __device__ static RowPtr row(const DevMat& m, int64_t r) {
        return {m.q + r * (m.K / 2), nullptr, m.s + r * (m.K / 32) * 2, nullptr};
    }
    __device__ static Raw load(const RowPtr& p, int s) {
        Raw w;
        w.q = gload_u4(p.q + 16 * (int64_t)s);
        w.d = *gptr((const uint16_t*)(p.s + 2 * s));
        return w;
    }
    // sum x (n - 8): nibble n of byte j is element j (low) or j + 16 (high)
    __device__ static float dot(const Raw& w, const float* xs, const float* x16, int s) {
        const float4* x4 = (const float4*)(xs + 32 * s);
        float t = -8.0f * (x16[2 * s] + x16[2 * s + 1]);
        const uint32_t q[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = q[i] & 0x0F0F0F0Fu, hi = (q[i] >> 4) & 0x0F0F0F0Fu;
            const float4 a = x4[i], b = x4[4 + i];
            t = fmaf(a.x, ub0(lo), t);
            t = fmaf(a.y, ub1(lo), t);
            t = fmaf(a.z, ub2(lo), t);
            t = fmaf(a.w, ub3(lo), t);
            t = fmaf(b.x, ub0(hi), t);
            t = fmaf(b.y, ub1(hi), t);
            t = fmaf(b.z, ub2(hi), t);
            t = fmaf(b.w, ub3(hi), t);
        }
        return h2f(w.d) * t;
    }
    __device__ static void dequant(const Raw& w, float* out) {
        const float d = h2f(w.d);
        const uint32_t q[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t byte = (q[j >> 2] >> (8 * (j & 3))) & 0xFFu;
            out[j] = d * (float)((int)(byte & 0x0F) - 8);
            out[j + 16] = d * (float)((int)(byte >> 4) - 8);
        }
    }
};

// ---------------------------------------------------------------- Q4_1
template <>
struct Fmt<TF_HIP_TYPE_Q4_1> {
    static constexpr int E = 32;
    static constexpr bool kNeedSums = true;
    struct Raw {
        uint4 q;
        uint32_t dm;  // d in the low half, m in the high half
    };
    __device__ static RowPtr row(const DevMat& m, int64_t r) {
        return {m.q + r * (m.K / 2), nullptr, m.s + r * (m.K / 32) * 4, nullptr};
    }
    __device__ static Raw load(const RowPtr& p, int s) {
        Raw w;
        w.q = gload_u4(p.q + 16 * (int64_t)s);
        w.dm = *gptr((const uint32_t*)(p.s + 4 * s));
        return w;
    }
    // sum x (n d + m) = d sum x n + m sum x
    __device__ static float dot(const Raw& w, const float* xs, const float* x16, int s) {
        const float4* x4 = (const float4*)(xs + 32 * s);
        float t = 0.0f;
        const uint32_t q[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = q[i] & 0x0F0F0F0Fu, hi = (q[i] >> 4) & 0x0F0F0F0Fu;
            const float4 a = x4[i], b = x4[4 + i];
            t = fmaf(a.x, ub0(lo), t);
            t = fmaf(a.y, ub1(lo), t);
            t = fmaf(a.z, ub2(lo), t);
            t = fmaf(a.w, ub3(lo), t);
            t = fmaf(b.x, ub0(hi), t);
            t = fmaf(b.y, ub1(hi), t);
            t = fmaf(b.z, ub2(hi), t);
            t = fmaf(b.w, ub3(hi), t);
        }
        return fmaf(h2f(w.dm & 0xFFFFu), t, h2f(w.dm >> 16) * (x16[2 * s] + x16[2 * s + 1]));
    }
    __device__ static void dequant(const Raw& w, float* out) {
        const float d = h2f(w.dm & 0xFFFFu), m = h2f(w.dm >> 16);
        const uint32_t q[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t byte = (q[j >> 2] >> (8 * (j & 3))) & 0xFFu;
            out[j] = (float)(byte & 0x0F) * d + m;
            out[j + 16] = (float)(byte >> 4) * d + m;
        }
    }
};

// ---------------------------------------------------------------- Q6_K
// 32-element group c of a row: lo[16] (element j low nibble, j+16 high nibble), hi[8]
// (byte j: elements j, j+8, j+16, j+24 at bits 0-1, 2-3, 4-5, 6-7), scales sc[2c],
// sc[2c+1] for elements 0-15 and 16-31, super-block scale d every 8 groups.
template <>
struct Fmt<TF_HIP_TYPE_Q6_K> {
    static constexpr int E = 32;
    static constexpr bool kNeedSums = true;
    struct Raw {
        uint4 lo;
        uint2 hi;
        uint32_t sc;  // two int8 scales in the low 16 bits
        uint32_t d;
    };
    __device__ static RowPtr row(const DevMat& m, int64_t r) {
        return {m.q + r * (m.K / 2), m.q2 + r * (m.K / 4), m.s + r * (m.K / 16), m.s2 + r * (m.K / 256) * 2};
    }
    __device__ static Raw load(const RowPtr& p, int s) {
        Raw w;
        w.lo = gload_u4(p.q + 16 * (int64_t)s);
        w.hi = gload_u2(p.q2 + 8 * (int64_t)s);
        w.sc = *gptr((const uint16_t*)(p.s + 2 * s));
        w.d = *gptr((const uint16_t*)(p.s2 + 2 * (s >> 3)));
        return w;
    }
    // 6-bit values u = lo4 | hi2 << 4 of elements 4i..4i+3 (first) and 16+4i.. (second)
    __device__ static void unpack(const Raw& w, int i, uint32_t& ua, uint32_t& ub) {
        const uint32_t l = i == 0 ? w.lo.x : i == 1 ? w.lo.y : i == 2 ? w.lo.z : w.lo.w;
        const uint32_t h = (i & 1) ? w.hi.y : w.hi.x;
        const int sh = 2 * (i >> 1);
        ua = (l & 0x0F0F0F0Fu) | (((h >> sh) & 0x03030303u) << 4);
        ub = ((l >> 4) & 0x0F0F0F0Fu) | (((h >> (sh + 4)) & 0x03030303u) << 4);
    }
    __device__ static float dot(const Raw& w, const float* xs, const float* x16, int s) {
        const float4* x4 = (const float4*)(xs + 32 * s);
        float t0 = -32.0f * x16[2 * s], t1 = -32.0f * x16[2 * s + 1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t ua, ub;
            unpack(w, i, ua, ub);
            const float4 a = x4[i], b = x4[4 + i];
            t0 = fmaf(a.x, ub0(ua), t0);
            t0 = fmaf(a.y, ub1(ua), t0);
            t0 = fmaf(a.z, ub2(ua), t0);
            t0 = fmaf(a.w, ub3(ua), t0);
            t1 = fmaf(b.x, ub0(ub), t1);
            t1 = fmaf(b.y, ub1(ub), t1);
            t1 = fmaf(b.z, ub2(ub), t1);
            t1 = fmaf(b.w, ub3(ub), t1);
        }
        const float sc0 = (float)(int8_t)(w.sc & 0xFFu), sc1 = (float)(int8_t)((w.sc >> 8) & 0xFFu);
        return h2f(w.d) * fmaf(sc0, t0, sc1 * t1);
    }
    __device__ static void dequant(const Raw& w, float* out) {
        const float d = h2f(w.d);
        const float sc0 = (float)(int8_t)(w.sc & 0xFFu), sc1 = (float)(int8_t)((w.sc >> 8) & 0xFFu);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t ua, ub;
            unpack(w, i, ua, ub);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                out[4 * i + j] = d * sc0 * (float)((int)((ua >> (8 * j)) & 0xFFu) - 32);
                out[16 + 4 * i + j] = d * sc1 * (float)((int)((ub >> (8 * j)) & 0xFFu) - 32);
            }
        }
    }
};

// ---------------------------------------------------------------- F16
template <>
struct Fmt<TF_HIP_TYPE_F16> {
    static constexpr int E = 8;
    static constexpr bool kNeedSums = false;
    struct Raw {
        uint4 q;
    };
    __device__ static RowPtr row(const DevMat& m, int64_t r) { return {m.q + r * m.K * 2, nullptr, nullptr, nullptr}; }
    __device__ static Raw load(const RowPtr& p, int s) { return {gload_u4(p.q + 16 * (int64_t)s)}; }
    __device__ static float dot(const Raw& w, const float* xs, const float*, int s) {
        const float4* x4 = (const float4*)(xs + 8 * s);
        const float4 a = x4[0], b = x4[1];
        float t = a.x * h2f(w.q.x & 0xFFFFu);
        t = fmaf(a.y, h2f(w.q.x >> 16), t);
        t = fmaf(a.z, h2f(w.q.y & 0xFFFFu), t);
        t = fmaf(a.w, h2f(w.q.y >> 16), t);
        t = fmaf(b.x, h2f(w.q.z & 0xFFFFu), t);
        t = fmaf(b.y, h2f(w.q.z >> 16), t);
        t = fmaf(b.z, h2f(w.q.w & 0xFFFFu), t);
        t = fmaf(b.w, h2f(w.q.w >> 16), t);
        return t;
    }
    __device__ static void dequant(const Raw& w, float* out) {
        const uint32_t q[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) out[i] = h2f((q[i >> 1] >> (16 * (i & 1))) & 0xFFFFu);
    }
};

// ---------------------------------------------------------------- F32
template <>
struct Fmt<TF_HIP_TYPE_F32> {
    static constexpr int E = 4;
    static constexpr bool kNeedSums = false;
    struct Raw {
        float4 q;
    };
    __device__ static RowPtr row(const DevMat& m, int64_t r) { return {m.q + r * m.K * 4, nullptr, nullptr, nullptr}; }
    __device__ static Raw load(const RowPtr& p, int s) { return {gload_f4(p.q + 16 * (int64_t)s)}; }
    __device__ static float dot(const Raw& w, const float* xs, const float*, int s) {
        const float4 a = *(const float4*)(xs + 4 * s);
        float t = a.x * w.q.x;
        t = fmaf(a.y, w.q.y, t);
        t = fmaf(a.z, w.q.z, t);
        t = fmaf(a.w, w.q.w, t);
        return t;
    }
    __device__ static void dequant(const Raw& w, float* out) {
        out[0] = w.q.x;
        out[1] = w.q.y;
        out[2] = w.q.z;
        out[3] = w.q.w;
    }
};

// Elements per step by runtime type (0 for unsupported).
__host__ __device__ inline int fmt_step_elems(int t) {
    switch (t) {
        case TF_HIP_TYPE_Q8_0: return 16;
        case TF_HIP_TYPE_Q4_0:
        case TF_HIP_TYPE_Q4_1:
        case TF_HIP_TYPE_Q6_K: return 32;
        case TF_HIP_TYPE_F16: return 8;
        case TF_HIP_TYPE_F32: return 4;
    }
    return 0;
}

}  // namespace tfk
