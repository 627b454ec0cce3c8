/*
 * oracle.c - CPU restatement of tinferno's --stage v2 token loop.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the oracle the HIP backend is checked
 * against, and the CPU baseline's restated form; never linked into the product.
 *
 * Built with -O3 -mavx2 -mfma -mf16c -ffp-contract=off: the only fused
 * multiply-adds are the explicit fmaf() calls, placed where g++ -O3 -mfma fuses
 * the reference's source. Sums keep the reference's association (the 8-lane AVX2
 * accumulator of quant.cpp:271-283 and its hsum8 of quant.cpp:186-195).
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

/* ------------------------------------------------------------------ formats */

/* quant.cpp:16-45. The reference's AVX2 build uses F16C (exact); signalling NaNs come back quiet. */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1F;
    uint32_t m = h & 0x3FF;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            e = 127 - 14;
            while ((m & 0x400) == 0) {
                m <<= 1;
                --e;
            }
            m &= 0x3FF;
            bits = sign | (e << 23) | (m << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13) | (m ? 0x00400000u : 0u);
    } else {
        bits = sign | ((e + (127 - 15)) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static int blck_size(int t) {
    switch (t) {
        case ORC_Q4_0: case ORC_Q4_1: case ORC_Q8_0: return 32;
        case ORC_Q6_K: return 256;
        case ORC_F32: case ORC_F16: return 1;
    }
    return 0;
}

static int blck_nbytes(int t) {
    switch (t) {
        case ORC_F32: return 4;
        case ORC_F16: return 2;
        case ORC_Q4_0: return 18;
        case ORC_Q4_1: return 20;
        case ORC_Q8_0: return 34;
        case ORC_Q6_K: return 210;
    }
    return 0;
}

/* tensor.cpp:66-70 */
int64_t orc_row_nbytes(int t, int64_t ne0) {
    const int bs = blck_size(t);
    if (bs == 0 || ne0 < 0 || ne0 % bs) return -1;
    return ne0 / bs * blck_nbytes(t);
}

static uint16_t rd16(const uint8_t* p) {
    uint16_t v;
    memcpy(&v, p, 2);
    return v;
}

/* quant.cpp:66-131: every product below is exact in fp32, so the order does not matter */
int orc_dequant_row(int t, const void* row, int64_t n, float* out) {
    const uint8_t* p = (const uint8_t*)row;
    if (orc_row_nbytes(t, n) < 0) return -1;
    switch (t) {
        case ORC_F32: memcpy(out, p, (size_t)n * 4); return 0;
        case ORC_F16:
            for (int64_t i = 0; i < n; ++i) out[i] = orc_f16_to_f32(rd16(p + 2 * i));
            return 0;
        case ORC_Q8_0:
            for (int64_t b = 0; b < n / 32; ++b, p += 34) {
                const float d = orc_f16_to_f32(rd16(p));
                for (int j = 0; j < 32; ++j) out[32 * b + j] = d * (float)(int8_t)p[2 + j];
            }
            return 0;
        case ORC_Q4_0:
            for (int64_t b = 0; b < n / 32; ++b, p += 18) {
                const float d = orc_f16_to_f32(rd16(p));
                for (int j = 0; j < 16; ++j) {
                    out[32 * b + j] = d * (float)((p[2 + j] & 0x0F) - 8);
                    out[32 * b + j + 16] = d * (float)((p[2 + j] >> 4) - 8);
                }
            }
            return 0;
        case ORC_Q4_1:
            for (int64_t b = 0; b < n / 32; ++b, p += 20) {
                const float d = orc_f16_to_f32(rd16(p));
                const float m = orc_f16_to_f32(rd16(p + 2));
                for (int j = 0; j < 16; ++j) {
                    out[32 * b + j] = (float)(p[4 + j] & 0x0F) * d + m;
                    out[32 * b + j + 16] = (float)(p[4 + j] >> 4) * d + m;
                }
            }
            return 0;
        case ORC_Q6_K:
            /* quant.cpp:101-127: element 128h + 32k + l takes its low nibble from
             * ql[64h + l + 32(k&1)] (high nibble for k >= 2), bits 2k..2k+1 of
             * qh[32h + l] on top, minus 32, times d * scales[(128h + 32k + l) / 16]. */
            for (int64_t b = 0; b < n / 256; ++b, p += 210) {
                const uint8_t* ql = p;
                const uint8_t* qh = p + 128;
                const int8_t* sc = (const int8_t*)(p + 192);
                const float d = orc_f16_to_f32(rd16(p + 208));
                float* y = out + 256 * b;
                for (int h = 0; h < 2; ++h)
                    for (int k = 0; k < 4; ++k)
                        for (int l = 0; l < 32; ++l) {
                            const uint8_t lo = ql[64 * h + l + 32 * (k & 1)];
                            const int nib = k < 2 ? (lo & 0x0F) : (lo >> 4);
                            const int q = (nib | (((qh[32 * h + l] >> (2 * k)) & 3) << 4)) - 32;
                            const int e = 128 * h + 32 * k + l;
                            y[e] = d * (float)sc[e / 16] * (float)q;
                        }
            }
            return 0;
    }
    return -1;
}

/* quant.cpp:186-195: ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)) */
static inline float hsum8(const float* a) {
    const float l0 = a[0] + a[4], l1 = a[1] + a[5], l2 = a[2] + a[6], l3 = a[3] + a[7];
    return (l0 + l1) + (l2 + l3);
}

/* quant.cpp:198-214 (AVX2 branch): one 8-lane accumulator, 4 FMAs per 32 elements,
 * then 8 at a time, hsum8, scalar tail. The tail only runs when n % 8 != 0, which no
 * GGUF row (multiples of 32) or head_dim of the workloads reaches. */
float orc_dot_f32(const float* a, const float* b, int n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 32 <= n; i += 32)
        for (int j = 0; j < 32; j += 8)
            for (int l = 0; l < 8; ++l) acc[l] = fmaf(a[i + j + l], b[i + j + l], acc[l]);
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; ++l) acc[l] = fmaf(a[i + l], b[i + l], acc[l]);
    float s = hsum8(acc);
    for (; i < n; ++i) s = fmaf(a[i], b[i], s);
    return s;
}

/* quant.cpp:245-264 (AVX2 branch) */
static float dot_f16(const float* x, const uint8_t* w, int n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; ++l) acc[l] = fmaf(x[i + l], orc_f16_to_f32(rd16(w + 2 * (i + l))), acc[l]);
    float s = hsum8(acc);
    for (; i < n; ++i) s = fmaf(x[i], orc_f16_to_f32(rd16(w + 2 * i)), s);
    return s;
}

/* quant.cpp:266-285 (AVX2 branch): per block, 8-lane FMA over x*q, hsum8, sum = fma(d, h, sum) */
static float dot_q8_0(const float* x, const uint8_t* w, int n) {
    float sum = 0;
    for (int b = 0; b < n / 32; ++b, w += 34, x += 32) {
        const float d = orc_f16_to_f32(rd16(w));
        const int8_t* q = (const int8_t*)(w + 2);
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int j = 0; j < 32; j += 8)
            for (int l = 0; l < 8; ++l) acc[l] = fmaf(x[j + l], (float)q[j + l], acc[l]);
        sum = fmaf(d, hsum8(acc), sum);
    }
    return sum;
}

/* quant.cpp:323-348 (AVX2 branch): nibbles unpacked to q-8 (low nibbles first), then as Q8_0 */
static float dot_q4_0(const float* x, const uint8_t* w, int n) {
    float sum = 0;
    for (int b = 0; b < n / 32; ++b, w += 18, x += 32) {
        const float d = orc_f16_to_f32(rd16(w));
        float q[32];
        for (int j = 0; j < 16; ++j) {
            q[j] = (float)((w[2 + j] & 0x0F) - 8);
            q[j + 16] = (float)((w[2 + j] >> 4) - 8);
        }
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int j = 0; j < 32; j += 8)
            for (int l = 0; l < 8; ++l) acc[l] = fmaf(x[j + l], q[j + l], acc[l]);
        sum = fmaf(d, hsum8(acc), sum);
    }
    return sum;
}

/* matmul.cpp:5-20: dispatch on dtype; Q4_1 and Q6_K dequantize the row, then dot_f32 */
float orc_dot_row(int t, const float* x, const void* row, int64_t k) {
    const uint8_t* w = (const uint8_t*)row;
    switch (t) {
        case ORC_F32: return orc_dot_f32(x, (const float*)row, (int)k);
        case ORC_F16: return dot_f16(x, w, (int)k);
        case ORC_Q8_0: return dot_q8_0(x, w, (int)k);
        case ORC_Q4_0: return dot_q4_0(x, w, (int)k);
        default: {
            float* tmp = (float*)malloc((size_t)k * sizeof(float));
            if (!tmp) return NAN;
            orc_dequant_row(t, row, k, tmp);
            const float s = orc_dot_f32(x, tmp, (int)k);
            free(tmp);
            return s;
        }
    }
}

/* matmul.cpp:22-32 (gemm_naive): each C[m,n] is an independent row dot, so threading over n
 * does not change any value */
int orc_matmul(float* c, const float* a, int m, int t, const void* w, int64_t n, int64_t k, int n_threads) {
    const int64_t rb = orc_row_nbytes(t, k);
    if (rb < 0 || m < 0 || n < 0) return -1;
    const uint8_t* wb = (const uint8_t*)w;
    if (n_threads < 1) n_threads = 1;
    if (t == ORC_Q4_1 || t == ORC_Q6_K) {
#pragma omp parallel num_threads(n_threads)
        {
            float* tmp = (float*)malloc((size_t)k * sizeof(float));
#pragma omp for schedule(static)
            for (int64_t r = 0; r < n; ++r) {
                orc_dequant_row(t, wb + r * rb, k, tmp);
                for (int i = 0; i < m; ++i) c[(int64_t)i * n + r] = orc_dot_f32(a + (int64_t)i * k, tmp, (int)k);
            }
            free(tmp);
        }
        return 0;
    }
#pragma omp parallel for num_threads(n_threads) schedule(static)
    for (int64_t r = 0; r < n; ++r)
        for (int i = 0; i < m; ++i) c[(int64_t)i * n + r] = orc_dot_row(t, a + (int64_t)i * k, wb + r * rb, k);
    return 0;
}

/* ------------------------------------------------------------------ layers */

/* layers.cpp:7-12: fp64 sum of squares (x*x is exact in fp64), inv in fp32, out = (x*inv)*w */
void orc_rmsnorm(float* out, const float* x, const float* w, int n, float eps) {
    double ss = 0;
    for (int i = 0; i < n; ++i) ss += (double)x[i] * (double)x[i];
    const float inv = 1.0f / sqrtf((float)(ss / n) + eps);
    for (int i = 0; i < n; ++i) out[i] = x[i] * inv * w[i];
}

/* layers.cpp:14-19 */
void orc_silu_mul(float* g, const float* u, int n) {
    for (int i = 0; i < n; ++i) {
        const float v = g[i];
        g[i] = (v / (1.0f + expf(-v))) * u[i];
    }
}

/* layers.cpp:25-35 */
void orc_softmax(float* x, int n) {
    float m = x[0];
    for (int i = 1; i < n; ++i) m = (m < x[i]) ? x[i] : m;
    float s = 0;
    for (int i = 0; i < n; ++i) {
        x[i] = expf(x[i] - m);
        s += x[i];
    }
    const float inv = 1.0f / s;
    for (int i = 0; i < n; ++i) x[i] *= inv;
}

/* ------------------------------------------------------------------ attention */

/* attention.cpp:9-29 */
void orc_rope_freqs(float* freq, int n_rot, float theta, int llama3, float scale, float low_freq_f,
                    float high_freq_f, float orig_ctx) {
    const int d2 = n_rot / 2;
    for (int i = 0; i < d2; ++i) {
        float f = 1.0f / powf(theta, (float)(2 * i) / (float)n_rot);
        if (llama3) {
            const float wavelen = 2.0f * 3.14159265358979323846f / f;
            const float lo_wl = orig_ctx / low_freq_f;
            const float hi_wl = orig_ctx / high_freq_f;
            if (wavelen < hi_wl) {
            } else if (wavelen > lo_wl) {
                f /= scale;
            } else {
                const float smooth = (orig_ctx / wavelen - low_freq_f) / (high_freq_f - low_freq_f);
                f = fmaf(smooth, f, (1.0f - smooth) * f / scale); /* g++ fuses smooth * f */
            }
        }
        freq[i] = f;
    }
}

/* attention.cpp:31-46: NeoX pairs (i, i + hd/2); g++ fuses x0*c and x0*s (the x1 products round first) */
void orc_rope(float* x, int n_heads, int hd, int pos, const float* freq) {
    const int d2 = hd / 2;
    for (int h = 0; h < n_heads; ++h) {
        float* xh = x + (int64_t)h * hd;
        for (int i = 0; i < d2; ++i) {
            const float ang = (float)pos * freq[i];
            const float c = cosf(ang);
            const float s = sinf(ang);
            const float x0 = xh[i], x1 = xh[i + d2];
            xh[i] = fmaf(x0, c, -(x1 * s));
            xh[i + d2] = fmaf(x0, s, x1 * c);
        }
    }
}

static int64_t kv_off(int layout, int n_kv, int max_seq, int hd, int g, int p) {
    /* kvcache.cpp:21-29 within one layer */
    if (layout == 1) return ((int64_t)g * max_seq + p) * hd;
    return ((int64_t)p * n_kv + g) * hd;
}

/* attention.cpp:55-80 */
void orc_attn_decode(float* out, const float* q, const float* kc, const float* vc, int layout, int n_kv,
                     int max_seq, int n_heads, int hd, int n_pos, float* scores) {
    const int n_rep = n_heads / n_kv;
    const float scale = 1.0f / sqrtf((float)hd);
    for (int h = 0; h < n_heads; ++h) {
        const int g = h / n_rep;
        const float* qh = q + (int64_t)h * hd;
        for (int p = 0; p < n_pos; ++p) scores[p] = scale * orc_dot_f32(qh, kc + kv_off(layout, n_kv, max_seq, hd, g, p), hd);
        orc_softmax(scores, n_pos);
        float* oh = out + (int64_t)h * hd;
        memset(oh, 0, (size_t)hd * sizeof(float));
        for (int p = 0; p < n_pos; ++p) {
            const float* vp = vc + kv_off(layout, n_kv, max_seq, hd, g, p);
            const float a = scores[p];
            for (int d = 0; d < hd; ++d) oh[d] = fmaf(a, vp[d], oh[d]);
        }
    }
}

/* attention.cpp:82-111: causal attention over the chunk's own rows only */
void orc_attn_prefill(float* out, const float* q, const float* k, const float* v, int seq, int n_heads,
                      int n_kv, int hd, float* scores) {
    const int n_rep = n_heads / n_kv;
    const float scale = 1.0f / sqrtf((float)hd);
    for (int h = 0; h < n_heads; ++h) {
        const int g = h / n_rep;
        for (int i = 0; i < seq; ++i) {
            const float* qi = q + ((int64_t)i * n_heads + h) * hd;
            for (int j = 0; j <= i; ++j) scores[j] = scale * orc_dot_f32(qi, k + ((int64_t)j * n_kv + g) * hd, hd);
            orc_softmax(scores, i + 1);
            float* oi = out + ((int64_t)i * n_heads + h) * hd;
            memset(oi, 0, (size_t)hd * sizeof(float));
            for (int j = 0; j <= i; ++j) {
                const float* vj = v + ((int64_t)j * n_kv + g) * hd;
                const float a = scores[j];
                for (int d = 0; d < hd; ++d) oi[d] = fmaf(a, vj[d], oi[d]);
            }
        }
    }
}

/* sampler.cpp:8-13 */
int orc_argmax(const float* x, int n) {
    int b = 0;
    for (int i = 1; i < n; ++i)
        if (x[i] > x[b]) b = i;
    return b;
}

/* ------------------------------------------------------------------ sampler.cpp:15-52 */

typedef struct {
    uint32_t mt[624];
    int i;
} orc_mt19937;

static void mt_seed(orc_mt19937* m, uint32_t seed) {
    m->mt[0] = seed;
    for (int i = 1; i < 624; ++i) m->mt[i] = 1812433253u * (m->mt[i - 1] ^ (m->mt[i - 1] >> 30)) + (uint32_t)i;
    m->i = 624;
}

static uint32_t mt_next(orc_mt19937* m) {
    if (m->i >= 624) {
        for (int k = 0; k < 624; ++k) {
            const uint32_t y = (m->mt[k] & 0x80000000u) | (m->mt[(k + 1) % 624] & 0x7fffffffu);
            m->mt[k] = m->mt[(k + 397) % 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908b0dfu : 0u);
        }
        m->i = 0;
    }
    uint32_t y = m->mt[m->i++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
}

void orc_uniform_draws(uint32_t seed, int n, float* out) {
    orc_mt19937 m;
    mt_seed(&m, seed);
    for (int i = 0; i < n; ++i) {
        float r = (float)mt_next(&m) / 4294967296.0f;
        if (r >= 1.0f) r = nextafterf(1.0f, 0.0f);
        out[i] = r;
    }
}

typedef struct {
    float v;
    int32_t i;
} orc_vi;

static int cmp_desc(const void* a, const void* b) {
    const orc_vi* x = (const orc_vi*)a;
    const orc_vi* y = (const orc_vi*)b;
    if (x->v > y->v) return -1;
    if (x->v < y->v) return 1;
    return (x->i > y->i) - (x->i < y->i);
}

int orc_sample_logits(const float* logits, int n, float temperature, float top_p, float r, int32_t* sorted_idx,
                      float* probs, int* n_last) {
    if (temperature <= 0.0f) return orc_argmax(logits, n);
    orc_vi* o = (orc_vi*)malloc((size_t)n * sizeof(orc_vi));
    float* p = (float*)malloc((size_t)n * sizeof(float));
    for (int i = 0; i < n; ++i) {
        o[i].v = logits[i];
        o[i].i = i;
    }
    qsort(o, (size_t)n, sizeof(orc_vi), cmp_desc);
    const float m = o[0].v;
    float s = 0.0f;
    for (int i = 0; i < n; ++i) {
        p[i] = expf((o[i].v - m) / temperature);
        s += p[i];
    }
    for (int i = 0; i < n; ++i) p[i] /= s;
    int last = n;
    if (top_p < 1.0f) {
        float acc = 0.0f;
        last = 0;
        for (int i = 0; i < n; ++i) {
            acc += p[i];
            last = i + 1;
            if (acc >= top_p) break;
        }
        float z = 0.0f;
        for (int i = 0; i < last; ++i) z += p[i];
        for (int i = 0; i < last; ++i) p[i] /= z;
    }
    int tok = o[last - 1].i;
    float acc = 0.0f;
    for (int i = 0; i < last; ++i) {
        acc += p[i];
        if (r <= acc) {
            tok = o[i].i;
            break;
        }
    }
    if (sorted_idx)
        for (int i = 0; i < n; ++i) sorted_idx[i] = o[i].i;
    if (probs) memcpy(probs, p, (size_t)n * sizeof(float));
    if (n_last) *n_last = last;
    free(o);
    free(p);
    return tok;
}

/* ------------------------------------------------------------------ GGUF (gguf.cpp:88-168) */

typedef struct {
    char name[96];
    int type, ndim;
    int64_t ne[4];
    uint64_t off;
    const uint8_t* data;
} orc_tensor;

typedef struct {
    char key[96];
    int kind; /* 0 int, 1 float, 2 string */
    uint64_t u;
    float f;
    char s[64];
} orc_kv;

struct orc_model {
    void* map;
    size_t map_size;
    int n_tensors, n_kvs;
    orc_tensor* tensors;
    orc_kv* kvs;
    char arch[32];
    char err[256];

    int n_vocab, n_embd, n_ff, n_layer, n_head, n_kv, hd, max_seq, layout, n_threads, n_pos;
    int bos, eos;
    float eps;
    float* freq;
    const orc_tensor *tok_embd, *out_norm, *output;
    const orc_tensor** lw; /* per layer: attn_norm q k v o bq bk bv ffn_norm gate up down */

    float *kc, *vc; /* [L][G*max_seq*hd] */
    int rows_cap;
    float *x, *xb, *q, *k, *v, *hb, *hb2, *att, *logits, *taps;
};

enum { LW_ANORM, LW_Q, LW_K, LW_V, LW_O, LW_BQ, LW_BK, LW_BV, LW_FNORM, LW_GATE, LW_UP, LW_DOWN, LW_N };

typedef struct {
    const uint8_t *p, *end;
    int bad;
} rd_t;

static int rd_need(rd_t* r, size_t n) {
    if (r->bad || (size_t)(r->end - r->p) < n) {
        r->bad = 1;
        return 0;
    }
    return 1;
}
static uint64_t rd_u(rd_t* r, size_t n) {
    uint64_t v = 0;
    if (!rd_need(r, n)) return 0;
    memcpy(&v, r->p, n);
    r->p += n;
    return v;
}
static const uint8_t* rd_str(rd_t* r, uint64_t* len) {
    *len = rd_u(r, 8);
    if (r->bad || *len > (uint64_t)(r->end - r->p)) {
        r->bad = 1;
        return NULL;
    }
    const uint8_t* s = r->p;
    r->p += *len;
    return s;
}
static size_t scalar_size(uint32_t t) {
    switch (t) {
        case 0: case 1: case 7: return 1;
        case 2: case 3: return 2;
        case 4: case 5: case 6: return 4;
        case 10: case 11: case 12: return 8;
    }
    return 0;
}
static void rd_skip(rd_t* r, uint32_t t) {
    uint64_t len;
    if (t == 8) {
        rd_str(r, &len);
    } else if (t == 9) {
        const uint32_t et = (uint32_t)rd_u(r, 4);
        const uint64_t n = rd_u(r, 8);
        for (uint64_t i = 0; i < n && !r->bad; ++i) rd_skip(r, et);
    } else if (scalar_size(t)) {
        if (rd_need(r, scalar_size(t))) r->p += scalar_size(t);
    } else {
        r->bad = 1;
    }
}

static const orc_kv* find_kv(const orc_model* m, const char* key) {
    for (int i = 0; i < m->n_kvs; ++i)
        if (!strcmp(m->kvs[i].key, key)) return &m->kvs[i];
    return NULL;
}
static uint64_t kv_u64(const orc_model* m, const char* key, uint64_t def) {
    const orc_kv* k = find_kv(m, key);
    return (k && k->kind == 0) ? k->u : def;
}
static float kv_f32(const orc_model* m, const char* key, float def) {
    const orc_kv* k = find_kv(m, key);
    return (k && k->kind == 1) ? k->f : def;
}
static const orc_tensor* find_t(const orc_model* m, const char* name) {
    for (int i = 0; i < m->n_tensors; ++i)
        if (!strcmp(m->tensors[i].name, name)) return &m->tensors[i];
    return NULL;
}

static int parse_gguf(orc_model* m, const char* path) {
    int fd = open(path, O_RDONLY);
    if (fd < 0) {
        snprintf(m->err, sizeof m->err, "cannot open %s", path);
        return -1;
    }
    struct stat st;
    fstat(fd, &st);
    m->map_size = (size_t)st.st_size;
    m->map = m->map_size ? mmap(NULL, m->map_size, PROT_READ, MAP_PRIVATE, fd, 0) : MAP_FAILED;
    close(fd);
    if (m->map == MAP_FAILED) {
        m->map = NULL;
        snprintf(m->err, sizeof m->err, "GGUF truncated");
        return -1;
    }
    rd_t r = {(const uint8_t*)m->map, (const uint8_t*)m->map + m->map_size, 0};
    if (rd_u(&r, 4) != 0x46554747u) {
        snprintf(m->err, sizeof m->err, "not a GGUF file: %s", path);
        return -1;
    }
    const uint32_t ver = (uint32_t)rd_u(&r, 4);
    if (ver != 2 && ver != 3) {
        snprintf(m->err, sizeof m->err, "unsupported GGUF version");
        return -1;
    }
    const uint64_t nt = rd_u(&r, 8), nkv = rd_u(&r, 8);
    if (r.bad || nt > 100000 || nkv > 100000) {
        snprintf(m->err, sizeof m->err, "GGUF truncated");
        return -1;
    }
    m->kvs = (orc_kv*)calloc(nkv + 1, sizeof(orc_kv));
    m->tensors = (orc_tensor*)calloc(nt + 1, sizeof(orc_tensor));
    for (uint64_t i = 0; i < nkv && !r.bad; ++i) {
        uint64_t len;
        const uint8_t* key = rd_str(&r, &len);
        const uint32_t t = (uint32_t)rd_u(&r, 4);
        if (r.bad) break;
        orc_kv* kv = &m->kvs[m->n_kvs];
        const int keep = len < sizeof kv->key;
        if (keep) memcpy(kv->key, key, len);
        switch (t) {
            case 0: case 2: case 4: case 10: kv->kind = 0; kv->u = rd_u(&r, scalar_size(t)); break;
            case 1: kv->kind = 0; kv->u = (uint64_t)(int64_t)(int8_t)rd_u(&r, 1); break;
            case 3: kv->kind = 0; kv->u = (uint64_t)(int64_t)(int16_t)rd_u(&r, 2); break;
            case 5: kv->kind = 0; kv->u = (uint64_t)(int64_t)(int32_t)rd_u(&r, 4); break;
            case 11: kv->kind = 0; kv->u = rd_u(&r, 8); break;
            case 6: {
                const uint32_t b = (uint32_t)rd_u(&r, 4);
                kv->kind = 1;
                memcpy(&kv->f, &b, 4);
                break;
            }
            case 12: {
                const uint64_t b = rd_u(&r, 8);
                double d;
                memcpy(&d, &b, 8);
                kv->kind = 1;
                kv->f = (float)d;
                break;
            }
            case 8: {
                uint64_t sl;
                const uint8_t* s = rd_str(&r, &sl);
                kv->kind = 2;
                if (s) memcpy(kv->s, s, sl < sizeof kv->s - 1 ? sl : sizeof kv->s - 1);
                break;
            }
            case 9: {
                const uint32_t et = (uint32_t)rd_u(&r, 4);
                const uint64_t n = rd_u(&r, 8);
                kv->kind = 0;
                kv->u = n; /* arrays: keep only the length (vocab fallback, model.cpp:15) */
                for (uint64_t j = 0; j < n && !r.bad; ++j) rd_skip(&r, et);
                break;
            }
            default: r.bad = 1;
        }
        if (keep) m->n_kvs++;
    }
    if (r.bad) {
        snprintf(m->err, sizeof m->err, "GGUF truncated");
        return -1;
    }
    const orc_kv* a = find_kv(m, "general.architecture");
    snprintf(m->arch, sizeof m->arch, "%s", (a && a->kind == 2) ? a->s : "llama");
    uint64_t align = kv_u64(m, "general.alignment", 32);
    if (!align) align = 32;
    for (uint64_t i = 0; i < nt && !r.bad; ++i) {
        orc_tensor* t = &m->tensors[i];
        uint64_t len;
        const uint8_t* nm = rd_str(&r, &len);
        if (nm) memcpy(t->name, nm, len < sizeof t->name - 1 ? len : sizeof t->name - 1);
        t->ndim = (int)rd_u(&r, 4);
        if (t->ndim < 1 || t->ndim > 4) {
            snprintf(m->err, sizeof m->err, "bad ndim for %s", t->name);
            return -1;
        }
        for (int d = 0; d < 4; ++d) t->ne[d] = d < t->ndim ? (int64_t)rd_u(&r, 8) : 1;
        t->type = (int)rd_u(&r, 4);
        if (blck_size(t->type) == 0) {
            snprintf(m->err, sizeof m->err, "unsupported ggml type %d", t->type);
            return -1;
        }
        t->off = rd_u(&r, 8);
        m->n_tensors++;
    }
    if (r.bad) {
        snprintf(m->err, sizeof m->err, "GGUF truncated");
        return -1;
    }
    const size_t hdr = (size_t)(r.p - (const uint8_t*)m->map);
    const size_t data_off = (hdr + align - 1) / align * align;
    for (int i = 0; i < m->n_tensors; ++i) {
        orc_tensor* t = &m->tensors[i];
        const int64_t rb = orc_row_nbytes(t->type, t->ne[0]);
        if (rb < 0) {
            snprintf(m->err, sizeof m->err, "row length not divisible by block size");
            return -1;
        }
        const size_t nb = (size_t)rb * (size_t)(t->ne[1] * t->ne[2] * t->ne[3]);
        const size_t abs_off = data_off + t->off;
        if (abs_off > m->map_size || nb > m->map_size - abs_off) {
            snprintf(m->err, sizeof m->err, "tensor out of range: %s", t->name);
            return -1;
        }
        t->data = (const uint8_t*)m->map + abs_off;
    }
    return 0;
}

/* ------------------------------------------------------------------ model (model.cpp) */

static char* key_of(char* buf, size_t n, const orc_model* m, const char* field) {
    snprintf(buf, n, "%s.%s", m->arch, field);
    return buf;
}

void orc_close(orc_model* m) {
    if (!m) return;
    if (m->map) munmap(m->map, m->map_size);
    free(m->kvs);
    free(m->tensors);
    free(m->freq);
    free(m->lw);
    free(m->kc);
    free(m->vc);
    free(m->x);
    free(m->xb);
    free(m->q);
    free(m->k);
    free(m->v);
    free(m->hb);
    free(m->hb2);
    free(m->att);
    free(m->logits);
    free(m->taps);
    free(m);
}

static int grow_rows(orc_model* m, int rows) {
    if (rows <= m->rows_cap) return 0;
    const int64_t D = m->n_embd, H = (int64_t)m->n_head * m->hd, KV = (int64_t)m->n_kv * m->hd, F = m->n_ff;
    free(m->x); free(m->xb); free(m->q); free(m->k); free(m->v); free(m->hb); free(m->hb2);
    m->x = (float*)calloc((size_t)(rows * D), 4);
    m->xb = (float*)calloc((size_t)(rows * (D > H ? D : H)), 4);
    m->q = (float*)calloc((size_t)(rows * (H > D ? H : D)), 4);
    m->k = (float*)calloc((size_t)(rows * KV), 4);
    m->v = (float*)calloc((size_t)(rows * KV), 4);
    m->hb = (float*)calloc((size_t)(rows * F), 4);
    m->hb2 = (float*)calloc((size_t)(rows * F), 4);
    if (!m->x || !m->xb || !m->q || !m->k || !m->v || !m->hb || !m->hb2) {
        snprintf(m->err, sizeof m->err, "out of memory");
        m->rows_cap = 0;
        return -1;
    }
    m->rows_cap = rows;
    return 0;
}

orc_model* orc_open(const char* path, int max_seq, int kv_layout, int n_threads, char* err, int err_len) {
    orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
    char kb[160];
    if (parse_gguf(m, path) != 0) goto fail;
    m->n_vocab = (int)kv_u64(m, key_of(kb, sizeof kb, m, "vocab_size"), 0);
    if (!m->n_vocab) m->n_vocab = (int)kv_u64(m, "tokenizer.ggml.tokens", 0);
    m->n_embd = (int)kv_u64(m, key_of(kb, sizeof kb, m, "embedding_length"), 0);
    m->n_ff = (int)kv_u64(m, key_of(kb, sizeof kb, m, "feed_forward_length"), 0);
    m->n_layer = (int)kv_u64(m, key_of(kb, sizeof kb, m, "block_count"), 0);
    m->n_head = (int)kv_u64(m, key_of(kb, sizeof kb, m, "attention.head_count"), 0);
    m->n_kv = (int)kv_u64(m, key_of(kb, sizeof kb, m, "attention.head_count_kv"), (uint64_t)m->n_head);
    m->hd = m->n_head ? m->n_embd / m->n_head : 0; /* model.cpp:22-24: n_embd/n_head wins */
    m->eps = kv_f32(m, key_of(kb, sizeof kb, m, "attention.layer_norm_rms_epsilon"), 1e-5f);
    {
        const float theta = kv_f32(m, key_of(kb, sizeof kb, m, "rope.freq_base"), 10000.0f);
        const orc_kv* st = find_kv(m, key_of(kb, sizeof kb, m, "rope.scaling.type"));
        const int llama3 = st && st->kind == 2 && !strcmp(st->s, "llama3");
        float sc = 1, lo = 1, hi = 4, oc = 8192;
        if (llama3) {
            sc = kv_f32(m, key_of(kb, sizeof kb, m, "rope.scaling.factor"), 32.0f);
            lo = kv_f32(m, key_of(kb, sizeof kb, m, "rope.scaling.low_freq_factor"), 1.0f);
            hi = kv_f32(m, key_of(kb, sizeof kb, m, "rope.scaling.high_freq_factor"), 4.0f);
            oc = (float)kv_u64(m, key_of(kb, sizeof kb, m, "rope.scaling.original_context_length"), 8192);
        }
        m->freq = (float*)calloc((size_t)(m->hd / 2 + 1), 4);
        orc_rope_freqs(m->freq, m->hd, theta, llama3, sc, lo, hi, oc);
    }
    m->bos = (int)kv_u64(m, "tokenizer.ggml.bos_token_id", 1);
    m->eos = (int)kv_u64(m, "tokenizer.ggml.eos_token_id", 2);
    if (!(m->tok_embd = find_t(m, "token_embd.weight"))) {
        snprintf(m->err, sizeof m->err, "missing tensor token_embd.weight");
        goto fail;
    }
    if (!(m->out_norm = find_t(m, "output_norm.weight"))) {
        snprintf(m->err, sizeof m->err, "missing tensor output_norm.weight");
        goto fail;
    }
    m->output = find_t(m, "output.weight");
    if (!m->output) m->output = m->tok_embd;
    if (!m->n_vocab) m->n_vocab = (int)m->tok_embd->ne[1];
    if (m->n_layer <= 0 || m->n_embd <= 0 || m->n_head <= 0 || m->n_kv <= 0 || m->n_head % m->n_kv) {
        snprintf(m->err, sizeof m->err, "bad hyperparameters");
        goto fail;
    }
    m->lw = (const orc_tensor**)calloc((size_t)m->n_layer * LW_N, sizeof(void*));
    for (int l = 0; l < m->n_layer; ++l) {
        static const char* names[LW_N] = {"attn_norm.weight", "attn_q.weight",   "attn_k.weight",
                                          "attn_v.weight",    "attn_output.weight", "attn_q.bias",
                                          "attn_k.bias",      "attn_v.bias",     "ffn_norm.weight",
                                          "ffn_gate.weight",  "ffn_up.weight",   "ffn_down.weight"};
        for (int j = 0; j < LW_N; ++j) {
            char nm[96];
            snprintf(nm, sizeof nm, "blk.%d.%s", l, names[j]);
            const orc_tensor* t = find_t(m, nm);
            const int optional = j == LW_BQ || j == LW_BK || j == LW_BV;
            if (!t && !optional) {
                snprintf(m->err, sizeof m->err, "missing tensor %s", nm);
                goto fail;
            }
            m->lw[l * LW_N + j] = t;
        }
    }
    m->max_seq = max_seq;
    m->layout = kv_layout;
    m->n_threads = n_threads > 0 ? n_threads : 1;
    {
        const size_t per_layer = (size_t)m->n_kv * (size_t)max_seq * (size_t)m->hd;
        m->kc = (float*)calloc(per_layer * (size_t)m->n_layer, 4);
        m->vc = (float*)calloc(per_layer * (size_t)m->n_layer, 4);
        m->att = (float*)calloc((size_t)max_seq + 1, 4);
        m->logits = (float*)calloc((size_t)m->n_vocab, 4);
        m->taps = (float*)calloc((size_t)(m->n_layer + 1) * (size_t)m->n_embd, 4);
        if (!m->kc || !m->vc || !m->att || !m->logits || !m->taps) {
            snprintf(m->err, sizeof m->err, "out of memory");
            goto fail;
        }
    }
    if (grow_rows(m, 1)) goto fail;
    return m;
fail:
    if (err && err_len > 0) snprintf(err, (size_t)err_len, "%s", m->err);
    orc_close(m);
    return NULL;
}

void orc_reset(orc_model* m) {
    const size_t n = (size_t)m->n_layer * m->n_kv * (size_t)m->max_seq * m->hd;
    m->n_pos = 0;
    memset(m->kc, 0, n * 4);
    memset(m->vc, 0, n * 4);
}

void orc_info(const orc_model* m, int32_t* o) {
    o[0] = m->n_vocab; o[1] = m->n_embd; o[2] = m->n_ff; o[3] = m->n_layer; o[4] = m->n_head;
    o[5] = m->n_kv; o[6] = m->hd; o[7] = m->n_pos; o[8] = m->max_seq; o[9] = m->layout;
}

float orc_rms_eps(const orc_model* m) { return m->eps; }
const char* orc_last_error(const orc_model* m) { return m->err; }

static float* layer_k(orc_model* m, int l) { return m->kc + (size_t)l * m->n_kv * m->max_seq * m->hd; }
static float* layer_v(orc_model* m, int l) { return m->vc + (size_t)l * m->n_kv * m->max_seq * m->hd; }

/* kvcache.cpp:31-36 */
static void kv_store(orc_model* m, int l, int pos, const float* k, const float* v) {
    for (int g = 0; g < m->n_kv; ++g) {
        const int64_t o = kv_off(m->layout, m->n_kv, m->max_seq, m->hd, g, pos);
        memcpy(layer_k(m, l) + o, k + (int64_t)g * m->hd, (size_t)m->hd * 4);
        memcpy(layer_v(m, l) + o, v + (int64_t)g * m->hd, (size_t)m->hd * 4);
    }
}

static void add_bias(float* x, const orc_tensor* b, int n) {
    /* model.cpp:85-89 reads the bias as raw F32 whatever its type */
    if (!b) return;
    const float* bp = (const float*)b->data;
    for (int i = 0; i < n; ++i) x[i] += bp[i];
}

static int mm(orc_model* m, float* c, const float* a, int rows, const orc_tensor* w) {
    return orc_matmul(c, a, rows, w->type, w->data, w->ne[1], w->ne[0], m->n_threads);
}

/* model.cpp:144-181 (seq == 1 with the cache path is model.cpp:108-142) */
static void layer_fwd(orc_model* m, int li, int seq, int decode) {
    const orc_tensor** L = m->lw + (size_t)li * LW_N;
    const int D = m->n_embd, H = m->n_head * m->hd, KV = m->n_kv * m->hd, F = m->n_ff;
    float* x = m->x;
    for (int i = 0; i < seq; ++i)
        orc_rmsnorm(m->xb + (int64_t)i * D, x + (int64_t)i * D, (const float*)L[LW_ANORM]->data, D, m->eps);
    mm(m, m->q, m->xb, seq, L[LW_Q]);
    mm(m, m->k, m->xb, seq, L[LW_K]);
    mm(m, m->v, m->xb, seq, L[LW_V]);
    for (int i = 0; i < seq; ++i) {
        add_bias(m->q + (int64_t)i * H, L[LW_BQ], H);
        add_bias(m->k + (int64_t)i * KV, L[LW_BK], KV);
        add_bias(m->v + (int64_t)i * KV, L[LW_BV], KV);
    }
    for (int i = 0; i < seq; ++i) {
        orc_rope(m->q + (int64_t)i * H, m->n_head, m->hd, m->n_pos + i, m->freq);
        orc_rope(m->k + (int64_t)i * KV, m->n_kv, m->hd, m->n_pos + i, m->freq);
    }
    for (int i = 0; i < seq; ++i) kv_store(m, li, m->n_pos + i, m->k + (int64_t)i * KV, m->v + (int64_t)i * KV);
    if (decode)
        orc_attn_decode(m->xb, m->q, layer_k(m, li), layer_v(m, li), m->layout, m->n_kv, m->max_seq, m->n_head,
                        m->hd, m->n_pos + 1, m->att);
    else
        orc_attn_prefill(m->xb, m->q, m->k, m->v, seq, m->n_head, m->n_kv, m->hd, m->att);
    mm(m, m->q, m->xb, seq, L[LW_O]);
    for (int64_t i = 0; i < (int64_t)seq * D; ++i) x[i] += m->q[i];
    for (int i = 0; i < seq; ++i)
        orc_rmsnorm(m->xb + (int64_t)i * D, x + (int64_t)i * D, (const float*)L[LW_FNORM]->data, D, m->eps);
    mm(m, m->hb, m->xb, seq, L[LW_GATE]);
    mm(m, m->hb2, m->xb, seq, L[LW_UP]);
    orc_silu_mul(m->hb, m->hb2, seq * F);
    mm(m, m->xb, m->hb, seq, L[LW_DOWN]);
    for (int64_t i = 0; i < (int64_t)seq * D; ++i) x[i] += m->xb[i];
    memcpy(m->taps + (size_t)li * D, x + (int64_t)(seq - 1) * D, (size_t)D * 4);
}

static int embed(orc_model* m, float* out, int32_t tok) {
    if (tok < 0 || tok >= m->tok_embd->ne[1]) {
        snprintf(m->err, sizeof m->err, "token %d out of range", tok);
        return -1;
    }
    const int64_t rb = orc_row_nbytes(m->tok_embd->type, m->tok_embd->ne[0]);
    return orc_dequant_row(m->tok_embd->type, m->tok_embd->data + (int64_t)tok * rb, m->n_embd, out);
}

static void head(orc_model* m, const float* xlast, float* logits) {
    const int D = m->n_embd;
    orc_rmsnorm(m->xb, xlast, (const float*)m->out_norm->data, D, m->eps);
    memcpy(m->taps + (size_t)m->n_layer * D, m->xb, (size_t)D * 4);
    mm(m, logits ? logits : m->logits, m->xb, 1, m->output);
}

int orc_prefill(orc_model* m, const int32_t* toks, int n, float* logits) {
    if (n <= 0) return 0;
    if (m->n_pos + n > m->max_seq) {
        snprintf(m->err, sizeof m->err, "prefill exceeds max_seq");
        return -1;
    }
    if (grow_rows(m, n)) return -1;
    for (int i = 0; i < n; ++i)
        if (embed(m, m->x + (int64_t)i * m->n_embd, toks[i])) return -1;
    for (int l = 0; l < m->n_layer; ++l) layer_fwd(m, l, n, 0);
    head(m, m->x + (int64_t)(n - 1) * m->n_embd, logits);
    m->n_pos += n;
    return 0;
}

int orc_decode(orc_model* m, int32_t tok, float* logits) {
    if (m->n_pos + 1 > m->max_seq) {
        snprintf(m->err, sizeof m->err, "decode exceeds max_seq");
        return -1;
    }
    if (embed(m, m->x, tok)) return -1;
    for (int l = 0; l < m->n_layer; ++l) layer_fwd(m, l, 1, 1);
    head(m, m->x, logits);
    m->n_pos += 1;
    return 0;
}

int orc_tap(const orc_model* m, int layer, float* out) {
    if (layer < 0 || layer > m->n_layer) return -1;
    memcpy(out, m->taps + (size_t)layer * m->n_embd, (size_t)m->n_embd * 4);
    return 0;
}

int orc_read_kv(const orc_model* m, int layer, int which, int pos0, int n, float* out) {
    if (layer < 0 || layer >= m->n_layer || pos0 < 0 || n < 0 || pos0 + n > m->max_seq) return -1;
    const float* base = (which ? m->vc : m->kc) + (size_t)layer * m->n_kv * m->max_seq * m->hd;
    for (int p = 0; p < n; ++p)
        for (int g = 0; g < m->n_kv; ++g)
            memcpy(out + ((int64_t)p * m->n_kv + g) * m->hd, base + kv_off(m->layout, m->n_kv, m->max_seq, m->hd, g, pos0 + p),
                   (size_t)m->hd * 4);
    return 0;
}
