/*
 * mi_oracle.c -- CPU restatement of mini-infer's layer-kernel arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product path).  See
 * mi_oracle.h for the contract of each function and the reference lines it
 * follows.  Built by oracle/Makefile into oracle/libmi_oracle.so.
 */
#include "mi_oracle.h"

#include <math.h>
#include <pthread.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* fp16 bit helpers                                                          */
/* ------------------------------------------------------------------------ */

static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* IEEE round-to-nearest-even fp32 -> fp16, including subnormals, overflow to
 * infinity and quiet NaN.  This is what the device's v_cvt_f16_f32 and the
 * reference kernels' __float2half do. */
uint16_t mio_f32_to_f16(float f) {
    const uint32_t u = f32_bits(f);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t absu = u & 0x7fffffffu;
    if (absu >= 0x7f800000u) {                       /* inf or nan */
        return (uint16_t)(sign | 0x7c00u | (absu > 0x7f800000u ? 0x200u : 0u));
    }
    if (absu >= 0x477ff000u) {                       /* >= 65520: rounds to inf */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (absu < 0x38800000u) {                        /* below 2^-14: subnormal */
        if (absu < 0x33000000u) return (uint16_t)sign; /* < 2^-25 -> 0 */
        /* value = sig * 2^(exp-150); target units of 2^-24. */
        const uint32_t exp = absu >> 23;
        const uint32_t sig = (absu & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - exp;           /* 150-24 = 126 */
        uint32_t q = sig >> shift;
        const uint32_t rem = sig & ((1u << shift) - 1u);
        const uint32_t halfway = 1u << (shift - 1u);
        if (rem > halfway || (rem == halfway && (q & 1u))) ++q;
        return (uint16_t)(sign | q);                 /* q may carry into min normal */
    }
    /* normal: rebias exponent (127 -> 15) and round 23 -> 10 mantissa bits */
    uint32_t v = absu - 0x38000000u;                 /* subtract (127-15) << 23 */
    const uint32_t rem = v & 0x1fffu;
    uint32_t q = v >> 13;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;
    return (uint16_t)(sign | q);                     /* carry may reach inf */
}

uint16_t mio_reftest_f32_to_f16(float f) {
    const uint32_t u = f32_bits(f);
    const uint32_t sign = (u >> 31) << 15;
    const uint32_t exp8 = (u >> 23) & 0xffu;
    const uint32_t man = u & 0x7fffffu;
    if (exp8 == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u));
    int32_t e = (int32_t)exp8 - 112;                 /* fp16 biased exponent */
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        /* full significand pre-shifted by (1 - e), then a further (13 - e)
         * with a half-unit added when bit (14 - e) is set */
        const uint32_t m = (man | 0x800000u) >> (uint32_t)(1 - e);
        const uint32_t sh = (uint32_t)(13 - e);
        const uint32_t q = (m + (((m >> (sh + 1u)) & 1u) << sh)) >> sh;
        return (uint16_t)(sign | (q & 0x3ffu));
    }
    /* a half-unit is added only when the kept LSB (bit 13) is odd */
    uint32_t q = (man + (((man >> 13) & 1u) << 12)) >> 13;
    if (q & 0x400u) { q = 0; e += 1; if (e > 31) e = 31; }
    return (uint16_t)(sign | ((uint32_t)e << 10) | (q & 0x3ffu));
}

void mio_reftest_f32_to_f16_array(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = mio_reftest_f32_to_f16(in[i]);
}

float mio_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    const uint32_t man = h & 0x3ffu;
    if (exp == 0x1fu) return bits_f32(sign | 0x7f800000u | (man << 13));
    if (exp == 0) {
        /* subnormal (or zero): man * 2^-24, exact in fp32 */
        const float mag = (float)man * 5.9604644775390625e-08f;
        return sign ? -mag : mag;
    }
    return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

void mio_f32_to_f16_array(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = mio_f32_to_f16(in[i]);
}

void mio_f16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = mio_f16_to_f32(in[i]);
}

/* ------------------------------------------------------------------------ */
/* Seeded generators (tests/test_helpers.h:46-68)                            */
/* ------------------------------------------------------------------------ */

static uint32_t xorshift32_step(uint32_t* s) {
    uint32_t x = *s;
    x ^= x << 13;
    x ^= x >> 17;
    x ^= x << 5;
    *s = x;
    return x;
}

void mio_fill_uniform(float* out, int64_t n, float scale, uint32_t seed) {
    uint32_t s = seed ? seed : 0x9E3779B9u;
    for (int64_t i = 0; i < n; ++i) {
        const uint32_t x = xorshift32_step(&s);
        /* 31 high bits as a fraction of 2^31, mapped to [-1, 1) */
        const float frac = (float)((x >> 1) & 0x7fffffffu) / 2147483648.0f;
        out[i] = (frac * 2.0f - 1.0f) * scale;
    }
}

void mio_fill_uniform_int64(int64_t* out, int64_t n, uint32_t seed,
                            int64_t lo, int64_t hi) {
    uint32_t s = seed ? seed : 0x12345678u;
    const uint32_t span = (uint32_t)(hi - lo + 1);
    for (int64_t i = 0; i < n; ++i) {
        const uint32_t x = xorshift32_step(&s);
        out[i] = lo + (int64_t)((x >> 1) % span);
    }
}

/* ------------------------------------------------------------------------ */
/* Row-parallel helper                                                       */
/* ------------------------------------------------------------------------ */

typedef void (*range_fn)(void* ctx, int64_t begin, int64_t end);

typedef struct {
    range_fn fn;
    void* ctx;
    int64_t begin, end;
} range_job;

static void* range_thread(void* p) {
    range_job* j = (range_job*)p;
    j->fn(j->ctx, j->begin, j->end);
    return NULL;
}

#define MIO_MAX_THREADS 256

static void parallel_for(range_fn fn, void* ctx, int64_t n, int nthreads) {
    if (nthreads > MIO_MAX_THREADS) nthreads = MIO_MAX_THREADS;
    if (nthreads <= 1 || n < 2 * nthreads) { fn(ctx, 0, n); return; }
    pthread_t tid[MIO_MAX_THREADS];
    range_job jobs[MIO_MAX_THREADS];
    const int64_t per = (n + nthreads - 1) / nthreads;
    int started = 0;
    for (int t = 0; t < nthreads; ++t) {
        const int64_t b = t * per;
        const int64_t e = b + per < n ? b + per : n;
        if (b >= e) break;
        jobs[t].fn = fn; jobs[t].ctx = ctx; jobs[t].begin = b; jobs[t].end = e;
        if (t == 0) continue;                 /* run slice 0 on this thread */
        if (pthread_create(&tid[t], NULL, range_thread, &jobs[t]) != 0) {
            range_thread(&jobs[t]);           /* no thread: run inline */
            tid[t] = 0;
        }
        started = t + 1;
    }
    fn(ctx, jobs[0].begin, jobs[0].end);
    for (int t = 1; t < started; ++t) if (tid[t]) pthread_join(tid[t], NULL);
}

/* ------------------------------------------------------------------------ */
/* RMSNorm and residual-add + RMSNorm                                        */
/* ------------------------------------------------------------------------ */

typedef struct {
    const uint16_t* x; uint16_t* residual; const uint16_t* w; float* y;
    int64_t D; float eps; int add_one; int fused;
} norm_ctx;

static void norm_rows(void* p, int64_t r0, int64_t r1) {
    const norm_ctx* c = (const norm_ctx*)p;
    const int64_t D = c->D;
    for (int64_t r = r0; r < r1; ++r) {
        const uint16_t* xr = c->x + r * D;
        uint16_t* rr = c->fused ? c->residual + r * D : NULL;
        float* yr = c->y + r * D;
        double ss = 0.0;
        for (int64_t i = 0; i < D; ++i) {
            float v = mio_f16_to_f32(xr[i]);
            if (c->fused) {
                /* residual add: fp32 sum of two fp16 values, rounded to fp16 */
                const uint16_t s = mio_f32_to_f16(mio_f16_to_f32(rr[i]) + v);
                rr[i] = s;
                v = mio_f16_to_f32(s);
            }
            yr[i] = v;                         /* stash the normed input */
            ss += (double)v * (double)v;
        }
        const float mean = (float)(ss / (double)D);
        const float rrms = (float)(1.0 / sqrt((double)mean + (double)c->eps));
        for (int64_t i = 0; i < D; ++i) {
            const float wv = mio_f16_to_f32(c->w[i]);
            const float f = c->add_one ? 1.0f + wv : wv;
            yr[i] = yr[i] * rrms * f;
        }
    }
}

void mio_rmsnorm(const uint16_t* x, const uint16_t* w, float* y,
                 int64_t N, int64_t D, float eps, int add_one, int nthreads) {
    norm_ctx c = {x, NULL, w, y, D, eps, add_one, 0};
    parallel_for(norm_rows, &c, N, nthreads);
}

void mio_fused_add_rmsnorm(const uint16_t* x, uint16_t* residual,
                           const uint16_t* w, float* y, int64_t N, int64_t D,
                           float eps, int add_one, int nthreads) {
    norm_ctx c = {x, residual, w, y, D, eps, add_one, 1};
    parallel_for(norm_rows, &c, N, nthreads);
}

/* ------------------------------------------------------------------------ */
/* RoPE                                                                      */
/* ------------------------------------------------------------------------ */

void mio_rope_inv_freq(float* inv_freq, int head_dim, float theta) {
    const int half = head_dim / 2;
    for (int i = 0; i < half; ++i) {
        const float e = (2.0f * (float)i) / (float)head_dim;
        inv_freq[i] = 1.0f / powf(theta, e);
    }
}

void mio_rope_tables(const float* inv_freq, const int64_t* positions,
                     uint16_t* cos_t, uint16_t* sin_t, int64_t N, int half) {
    for (int64_t n = 0; n < N; ++n) {
        const float pos = (float)positions[n];
        for (int i = 0; i < half; ++i) {
            const float ang = pos * inv_freq[i];
            /* double cos/sin rounded once to fp32 = correctly rounded cosf */
            const float c = (float)cos((double)ang);
            const float s = (float)sin((double)ang);
            cos_t[n * half + i] = mio_f32_to_f16(c);
            sin_t[n * half + i] = mio_f32_to_f16(s);
        }
    }
}

typedef struct {
    const uint16_t* x; const uint16_t* c; const uint16_t* s; float* y;
    int H; int hd;
} rope_ctx;

static void rope_rows(void* p, int64_t t0, int64_t t1) {
    const rope_ctx* k = (const rope_ctx*)p;
    const int half = k->hd / 2;
    for (int64_t t = t0; t < t1; ++t) {
        const uint16_t* cr = k->c + t * half;
        const uint16_t* sr = k->s + t * half;
        for (int h = 0; h < k->H; ++h) {
            const int64_t base = (t * k->H + h) * (int64_t)k->hd;
            for (int i = 0; i < half; ++i) {
                const float x1 = mio_f16_to_f32(k->x[base + i]);
                const float x2 = mio_f16_to_f32(k->x[base + half + i]);
                const float cv = mio_f16_to_f32(cr[i]);
                const float sv = mio_f16_to_f32(sr[i]);
                k->y[base + i] = x1 * cv - x2 * sv;
                k->y[base + half + i] = x2 * cv + x1 * sv;
            }
        }
    }
}

void mio_rope_neox(const uint16_t* x, const uint16_t* cos_t,
                   const uint16_t* sin_t, float* y, int64_t T, int H, int hd,
                   int nthreads) {
    rope_ctx c = {x, cos_t, sin_t, y, H, hd};
    parallel_for(rope_rows, &c, T, nthreads);
}

/* ------------------------------------------------------------------------ */
/* Gated activations                                                         */
/* ------------------------------------------------------------------------ */

static float silu_f(float g) { return g / (1.0f + expf(-g)); }

static float gelu_tanh_f(float x) {
    const float k0 = 0.7978845608028654f;      /* sqrt(2/pi) */
    const float k1 = 0.044715f;
    return 0.5f * x * (1.0f + tanhf(k0 * (x + k1 * x * x * x)));
}

typedef struct {
    const uint16_t* a; const uint16_t* b; float* out; int kind;
} ew_ctx;

enum { EW_SWIGLU = 0, EW_GELU = 1, EW_GEGLU = 2 };

static void ew_range(void* p, int64_t i0, int64_t i1) {
    const ew_ctx* c = (const ew_ctx*)p;
    for (int64_t i = i0; i < i1; ++i) {
        const float a = mio_f16_to_f32(c->a[i]);
        switch (c->kind) {
        case EW_SWIGLU: c->out[i] = silu_f(a) * mio_f16_to_f32(c->b[i]); break;
        case EW_GELU:   c->out[i] = gelu_tanh_f(a); break;
        default:        c->out[i] = gelu_tanh_f(a) * mio_f16_to_f32(c->b[i]); break;
        }
    }
}

void mio_swiglu(const uint16_t* g, const uint16_t* u, float* out, int64_t n,
                int nthreads) {
    ew_ctx c = {g, u, out, EW_SWIGLU};
    parallel_for(ew_range, &c, n, nthreads);
}

void mio_gelu_tanh(const uint16_t* x, float* y, int64_t n, int nthreads) {
    ew_ctx c = {x, NULL, y, EW_GELU};
    parallel_for(ew_range, &c, n, nthreads);
}

void mio_geglu(const uint16_t* g, const uint16_t* u, float* out, int64_t n,
               int nthreads) {
    ew_ctx c = {g, u, out, EW_GEGLU};
    parallel_for(ew_range, &c, n, nthreads);
}

void mio_geglu_composed(const uint16_t* g, const uint16_t* u, uint16_t* out,
                        int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        const uint16_t a = mio_f32_to_f16(gelu_tanh_f(mio_f16_to_f32(g[i])));
        out[i] = mio_f32_to_f16(mio_f16_to_f32(a) * mio_f16_to_f32(u[i]));
    }
}

void mio_add_inplace(uint16_t* y, const uint16_t* x, int64_t n) {
    for (int64_t i = 0; i < n; ++i)
        y[i] = mio_f32_to_f16(mio_f16_to_f32(y[i]) + mio_f16_to_f32(x[i]));
}

void mio_add_bias(uint16_t* y, const uint16_t* bias, int64_t M, int64_t N,
                  int64_t batch_stride) {
    if (M <= 0 || N <= 0) return;
    const int64_t batches = batch_stride / (M * N);
    for (int64_t b = 0; b < batches; ++b)
        for (int64_t m = 0; m < M; ++m)
            for (int64_t n = 0; n < N; ++n) {
                uint16_t* p = y + b * batch_stride + m * N + n;
                *p = mio_f32_to_f16(mio_f16_to_f32(*p) + mio_f16_to_f32(bias[n]));
            }
}

void mio_mul_inplace(uint16_t* y, const uint16_t* x, int64_t n) {
    for (int64_t i = 0; i < n; ++i)
        y[i] = mio_f32_to_f16(mio_f16_to_f32(y[i]) * mio_f16_to_f32(x[i]));
}

void mio_scale_inplace(uint16_t* y, float scale, int64_t n) {
    for (int64_t i = 0; i < n; ++i)
        y[i] = mio_f32_to_f16(mio_f16_to_f32(y[i]) * scale);
}

/* ------------------------------------------------------------------------ */
/* Softmax                                                                   */
/* ------------------------------------------------------------------------ */

typedef struct { const uint16_t* x; float* y; int64_t D; } sm_ctx;

static void softmax_rows(void* p, int64_t r0, int64_t r1) {
    const sm_ctx* c = (const sm_ctx*)p;
    for (int64_t r = r0; r < r1; ++r) {
        const uint16_t* xr = c->x + r * c->D;
        float* yr = c->y + r * c->D;
        float m = -INFINITY;
        for (int64_t i = 0; i < c->D; ++i) {
            const float v = mio_f16_to_f32(xr[i]);
            if (v > m) m = v;
        }
        double sum = 0.0;
        for (int64_t i = 0; i < c->D; ++i) {
            const double e = exp((double)mio_f16_to_f32(xr[i]) - (double)m);
            yr[i] = (float)e;
            sum += e;
        }
        const double inv = 1.0 / sum;
        for (int64_t i = 0; i < c->D; ++i) yr[i] = (float)((double)yr[i] * inv);
    }
}

void mio_softmax(const uint16_t* x, float* y, int64_t N, int64_t D,
                 int nthreads) {
    sm_ctx c = {x, y, D};
    parallel_for(softmax_rows, &c, N, nthreads);
}

/* ------------------------------------------------------------------------ */
/* Embedding gather                                                          */
/* ------------------------------------------------------------------------ */

typedef struct {
    const int64_t* ids; const uint16_t* table; uint16_t* out;
    int64_t H; int64_t vocab;
} gather_ctx;

static void gather_rows(void* p, int64_t t0, int64_t t1) {
    const gather_ctx* c = (const gather_ctx*)p;
    for (int64_t t = t0; t < t1; ++t) {
        const int64_t id = c->ids[t];
        uint16_t* dst = c->out + t * c->H;
        if (id < 0 || (c->vocab > 0 && id >= c->vocab)) {
            memset(dst, 0, (size_t)c->H * 2u);
        } else {
            memcpy(dst, c->table + id * c->H, (size_t)c->H * 2u);
        }
    }
}

void mio_embedding_gather(const int64_t* ids, const uint16_t* table,
                          uint16_t* out, int64_t T, int64_t H, int64_t vocab,
                          int nthreads) {
    gather_ctx c = {ids, table, out, H, vocab};
    parallel_for(gather_rows, &c, T, nthreads);
}

/* ------------------------------------------------------------------------ */
/* Paged KV scatter and greedy argmax                                        */
/* ------------------------------------------------------------------------ */

void mio_paged_kv_scatter(const uint16_t* src, uint16_t* cache, const int32_t* block_table,
                          const int32_t* seq_len, const int32_t* start_pos, int64_t B,
                          int64_t S, int64_t layer, int64_t num_blocks, int64_t H_kv, int64_t D,
                          int64_t block_size, int64_t max_blocks_per_seq) {
    for (int64_t b = 0; b < B; ++b) {
        for (int64_t s = 0; s < S; ++s) {
            const int64_t pos = (int64_t)start_pos[b] + s;
            if (pos < 0 || pos >= seq_len[b]) continue;
            const int64_t blk = pos / block_size;
            if (blk >= max_blocks_per_seq) continue;
            const int64_t phys = block_table[b * max_blocks_per_seq + blk];
            if (phys < 0 || phys >= num_blocks) continue;
            const int64_t slot = pos % block_size;
            for (int64_t h = 0; h < H_kv; ++h) {
                const uint16_t* from = src + ((b * S + s) * H_kv + h) * D;
                uint16_t* to = cache + ((layer * num_blocks + phys) * H_kv + h) * block_size * D
                               + slot * D;
                memcpy(to, from, (size_t)D * 2u);
            }
        }
    }
}

void mio_greedy_argmax(const uint16_t* logits, int64_t B, int64_t V, int32_t* out) {
    enum { BLOCK = 256 };
    float best_v[BLOCK];
    int32_t best_i[BLOCK];
    for (int64_t r = 0; r < B; ++r) {
        const uint16_t* row = logits + r * V;
        /* each "thread" keeps its first strict maximum over a stride-256 scan */
        for (int t = 0; t < BLOCK; ++t) {
            float m = -INFINITY;
            int32_t idx = -1;
            for (int64_t i = t; i < V; i += BLOCK) {
                const float v = mio_f16_to_f32(row[i]);
                if (v > m) { m = v; idx = (int32_t)i; }
            }
            best_v[t] = m;
            best_i[t] = idx;
        }
        /* tree reduction: the partner's value replaces only when strictly larger */
        for (int off = BLOCK / 2; off > 0; off >>= 1) {
            for (int t = 0; t < off; ++t) {
                if (best_v[t + off] > best_v[t]) {
                    best_v[t] = best_v[t + off];
                    best_i[t] = best_i[t + off];
                }
            }
        }
        out[r] = best_i[0];
    }
}

uint64_t mio_fmix64(uint64_t s) {
    s ^= s >> 33;
    s *= 0xff51afd7ed558ccdULL;
    s ^= s >> 33;
    s *= 0xc4ceb9fe1a85ec53ULL;
    s ^= s >> 33;
    return s;
}

void mio_top_p_sample(const uint16_t* logits, int64_t B, int64_t vocab, float p,
                      float temperature, uint64_t seed, int32_t* out) {
    enum { K = 256, STRIDE = 128 };
    if (vocab > 30000) {
        mio_greedy_argmax(logits, B, vocab, out);
        return;
    }
    for (int64_t r = 0; r < B; ++r) {
        const uint16_t* x = logits + r * vocab;
        float row_max = -INFINITY;
        for (int64_t i = 0; i < vocab; ++i) {
            const float v = mio_f16_to_f32(x[i]) / temperature;
            if (v > row_max) row_max = v;
        }
        double sum = 0.0;
        for (int64_t i = 0; i < vocab; ++i)
            sum += (double)expf(mio_f16_to_f32(x[i]) / temperature - row_max);
        const float row_sum = (float)sum;
        /* K selection rounds over the first thread's share: indices 0, 128, ... */
        int32_t top_idx[K];
        float top_val[K];
        for (int k = 0; k < K; ++k) {
            float best_val = -INFINITY;
            int32_t best_idx = -1;
            for (int64_t i = 0; i < vocab; i += STRIDE) {
                int used = 0;
                for (int j = 0; j < k; ++j)
                    if (top_idx[j] == (int32_t)i) { used = 1; break; }
                if (used) continue;
                const float v = expf(mio_f16_to_f32(x[i]) / temperature - row_max) / row_sum;
                if (v > best_val) { best_val = v; best_idx = (int32_t)i; }
            }
            top_idx[k] = best_idx;
            top_val[k] = best_val;
        }
        /* insertion sort, descending (stable) */
        for (int i = 1; i < K; ++i) {
            const float v = top_val[i];
            const int32_t ix = top_idx[i];
            int j = i - 1;
            while (j >= 0 && top_val[j] < v) {
                top_val[j + 1] = top_val[j];
                top_idx[j + 1] = top_idx[j];
                --j;
            }
            top_val[j + 1] = v;
            top_idx[j + 1] = ix;
        }
        const uint64_t rs = seed + (uint64_t)r;
        float cum = 0.0f;
        int32_t choice = top_idx[K - 1];
        for (int i = 0; i < K; ++i) {
            cum += top_val[i];
            if (cum >= p) {
                const uint64_t h = mio_fmix64(rs ^ ((uint64_t)(int64_t)top_idx[i] << 32));
                const float u = (float)(h & 0xFFFFFFu) / (float)0x1000000;
                int slot = (int)(u * (float)(i + 1));
                if (slot < 0) slot = 0;
                if (slot > i) slot = i;
                choice = top_idx[slot];
                break;
            }
        }
        out[r] = choice;
    }
}
