/*
 * cuca_oracle.c -- CPU restatement of the reference's per-layer ops.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker and the CPU-baseline timer.
 * Nothing in the product (cuca_amd/, libcuca_hip.so) links or loads it.
 * Build: oracle/build.py (gcc -O2 -ffp-contract=off -pthread).
 *
 * Each function names the reference file:line it follows; paths are under
 * src/provider/local/model/ of nassor/cuca 0.10.0.  Where the reference
 * calls candle 0.11.1 (not vendored in the reference), the restated
 * formula is the one the reference's own tests and GPU mirror state
 * (gpu.rs:5883-5913, moe_kernel.rs:2340-2352); the bit-level summation
 * order of candle's kernels is not pinned (see the tests' tolerances).
 */
#include "cuca_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* binary16 conversions                                                */
/* ------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0) {
        if (m == 0) return u2f(sign);
        /* subnormal: m * 2^-24, exact in f32 */
        float v = (float)m * 5.9604644775390625e-8f;
        return u2f(sign | f2u(v));
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t oracle_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf / nan (quiet the nan, keep top payload) */
        if (ax == 0x7f800000u) return sign | 0x7c00u;
        return sign | 0x7e00u | (uint16_t)((ax >> 13) & 0x3ffu);
    }
    uint32_t e = ax >> 23;
    uint32_t m = ax & 0x7fffffu;
    if (e < 113) { /* below 2^-14: f16 subnormal or zero */
        if (e == 0) return sign; /* f32 subnormal is far below half of 2^-24 */
        uint32_t M = m | 0x800000u;
        uint32_t s = 126u - e; /* >= 14 */
        if (s >= 25) return sign;
        uint32_t r = M >> s;
        uint32_t rem = M & ((1u << s) - 1u);
        uint32_t half = 1u << (s - 1u);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return sign | (uint16_t)r;
    }
    if (e > 142) return sign | 0x7c00u; /* >= 2^16: overflow */
    uint32_t h = ((e - 112u) << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++; /* carries into e */
    return sign | (uint16_t)h;
}

/* Bulk conversions, with the x86 F16C instructions when the CPU has them
 * (as the `half` crate's conversions do, by runtime detection): the same
 * values as the scalar restatement above -- exact widening, and rounding to
 * nearest-even with the MXCSR rounding overridden -- which the tests check
 * exhaustively for f16 -> f32 and over millions of f32 values. */
#if defined(__x86_64__)
#include <immintrin.h>
__attribute__((target("avx,f16c"))) static void h2f_f16c(const uint16_t *h, float *f, int64_t n) {
    int64_t i = 0;
    for (; i + 8 <= n; i += 8)
        _mm256_storeu_ps(f + i, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(h + i))));
    for (; i < n; i++) f[i] = oracle_f16_to_f32(h[i]);
}
__attribute__((target("avx,f16c"))) static void f2h_f16c(const float *f, uint16_t *h, int64_t n) {
    int64_t i = 0;
    for (; i + 8 <= n; i += 8)
        _mm_storeu_si128((__m128i *)(h + i),
                         _mm256_cvtps_ph(_mm256_loadu_ps(f + i), _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC));
    for (; i < n; i++) h[i] = oracle_f32_to_f16(f[i]);
}
static int have_f16c(void) {
    static int v = -1;
    if (v < 0) v = __builtin_cpu_supports("f16c") && __builtin_cpu_supports("avx") ? 1 : 0;
    return v;
}
#endif

void oracle_f16_to_f32_n(const uint16_t *h, float *f, int64_t n) {
#if defined(__x86_64__)
    if (have_f16c()) { h2f_f16c(h, f, n); return; }
#endif
    for (int64_t i = 0; i < n; i++) f[i] = oracle_f16_to_f32(h[i]);
}

void oracle_f32_to_f16_n(const float *f, uint16_t *h, int64_t n) {
#if defined(__x86_64__)
    if (have_f16c()) { f2h_f16c(f, h, n); return; }
#endif
    for (int64_t i = 0; i < n; i++) h[i] = oracle_f32_to_f16(f[i]);
}

/* The scalar restatement over n values (the tests compare both paths). */
void oracle_f16_to_f32_soft_n(const uint16_t *h, float *f, int64_t n) {
    for (int64_t i = 0; i < n; i++) f[i] = oracle_f16_to_f32(h[i]);
}

void oracle_f32_to_f16_soft_n(const float *f, uint16_t *h, int64_t n) {
    for (int64_t i = 0; i < n; i++) h[i] = oracle_f32_to_f16(f[i]);
}

int oracle_has_f16c(void) {
#if defined(__x86_64__)
    return have_f16c();
#else
    return 0;
#endif
}

static inline float load_el(const void *p, int64_t i, int dtype) {
    return dtype == OR_F16 ? oracle_f16_to_f32(((const uint16_t *)p)[i])
                           : ((const float *)p)[i];
}

static inline void store_el(void *p, int64_t i, float v, int dtype) {
    if (dtype == OR_F16) ((uint16_t *)p)[i] = oracle_f32_to_f16(v);
    else ((float *)p)[i] = v;
}

/* n values of a row starting at element `at`, widened to f32 / rounded back */
static void load_row(const void *p, int64_t at, int64_t n, int dtype, float *dst) {
    if (dtype == OR_F16) oracle_f16_to_f32_n((const uint16_t *)p + at, dst, n);
    else memcpy(dst, (const float *)p + at, sizeof(float) * (size_t)n);
}

static void store_row(void *p, int64_t at, int64_t n, int dtype, const float *src) {
    if (dtype == OR_F16) oracle_f32_to_f16_n(src, (uint16_t *)p + at, n);
    else memcpy((float *)p + at, src, sizeof(float) * (size_t)n);
}

/* ------------------------------------------------------------------ */
/* a tiny row-parallel for (the CPU-baseline's threading)              */
/* ------------------------------------------------------------------ */

typedef void (*range_fn)(void *ctx, int64_t begin, int64_t end);

/* A persistent pool: worker threads are started once, on the first
 * parallel call, and wait between calls (starting threads per call would
 * dominate a CPU timing of these memory-bound loops).  One call runs at a
 * time (the pool's lock is held for the whole call). */
#define POOL_MAX 256
static struct {
    pthread_mutex_t call_lock, mu;
    pthread_cond_t go, done;
    int started;            /* workers running */
    uint64_t generation;    /* bumped per call  */
    int active;             /* workers in this call (1..started) */
    int pending;            /* workers not finished yet */
    range_fn fn;
    void *ctx;
    int64_t n, per, extra;
} g_pool = {PTHREAD_MUTEX_INITIALIZER, PTHREAD_MUTEX_INITIALIZER, PTHREAD_COND_INITIALIZER,
            PTHREAD_COND_INITIALIZER, 0, 0, 0, 0, NULL, NULL, 0, 0, 0};

static void pool_chunk(int t, int64_t *b, int64_t *e) {
    int64_t per = g_pool.per, extra = g_pool.extra;
    *b = t * per + (t < extra ? t : extra);
    *e = *b + per + (t < extra ? 1 : 0);
}

static void *pool_worker(void *arg) {
    const int t = (int)(intptr_t)arg;  /* this worker runs chunk t (>= 1) */
    uint64_t seen = 0;
    pthread_mutex_lock(&g_pool.mu);
    for (;;) {
        while (g_pool.generation == seen) pthread_cond_wait(&g_pool.go, &g_pool.mu);
        seen = g_pool.generation;
        if (t >= g_pool.active) continue;
        range_fn fn = g_pool.fn;
        void *ctx = g_pool.ctx;
        int64_t b, e;
        pool_chunk(t, &b, &e);
        pthread_mutex_unlock(&g_pool.mu);
        if (b < e) fn(ctx, b, e);
        pthread_mutex_lock(&g_pool.mu);
        if (--g_pool.pending == 0) pthread_cond_signal(&g_pool.done);
    }
    return NULL;
}

/* Split rows [0, n) into nthreads contiguous chunks; chunk 0 runs on the
 * calling thread. */
static void parallel_rows(int nthreads, int64_t n, range_fn fn, void *ctx) {
    if (nthreads <= 1 || n < 2) { fn(ctx, 0, n); return; }
    if (nthreads > n) nthreads = (int)n;
    if (nthreads > POOL_MAX) nthreads = POOL_MAX;
    pthread_mutex_lock(&g_pool.call_lock);
    pthread_mutex_lock(&g_pool.mu);
    while (g_pool.started < nthreads - 1) {
        pthread_t th;
        if (pthread_create(&th, NULL, pool_worker, (void *)(intptr_t)(g_pool.started + 1)) != 0) break;
        pthread_detach(th);
        g_pool.started++;
    }
    const int active = g_pool.started + 1 < nthreads ? g_pool.started + 1 : nthreads;
    g_pool.fn = fn;
    g_pool.ctx = ctx;
    g_pool.n = n;
    g_pool.per = n / active;
    g_pool.extra = n % active;
    g_pool.active = active;
    g_pool.pending = active - 1;
    g_pool.generation++;
    pthread_cond_broadcast(&g_pool.go);
    int64_t b, e;
    pool_chunk(0, &b, &e);
    pthread_mutex_unlock(&g_pool.mu);
    fn(ctx, b, e);
    pthread_mutex_lock(&g_pool.mu);
    while (g_pool.pending > 0) pthread_cond_wait(&g_pool.done, &g_pool.mu);
    pthread_mutex_unlock(&g_pool.mu);
    pthread_mutex_unlock(&g_pool.call_lock);
}

/* ------------------------------------------------------------------ */
/* a1-a3: Q4_0 / Q8_0 dequant and the embedding gather                 */
/* ------------------------------------------------------------------ */

int64_t oracle_row_bytes(uint32_t ggml_type, int64_t hidden) {
    /* gguf/dtype.rs:195-250: Q4_0 = 18 B, Q8_0 = 34 B per 32 values */
    int64_t bs = ggml_type == OR_Q4_0 ? 18 : ggml_type == OR_Q8_0 ? 34 : -1;
    if (bs < 0 || hidden <= 0 || hidden % 32 != 0) return -1;
    return hidden / 32 * bs;
}

/* quant.rs:107-198, the Q4_0 and Q8_0 arms of dequant_ggml_row.  The scale
 * is folded into the block's f16 `d` first (quant.rs:121-123), then each
 * quant is multiplied by it: two f32 roundings, in that order. */
int oracle_dequant_row(uint32_t ggml_type, const uint8_t *bytes, int64_t nbytes,
                       float scale, float *out, int64_t n) {
    int64_t rb = oracle_row_bytes(ggml_type, n);
    if (rb < 0 || rb != nbytes) return -1;
    int64_t bs = ggml_type == OR_Q4_0 ? 18 : 34;
    for (int64_t b = 0; b < n / 32; b++) {
        const uint8_t *blk = bytes + b * bs;
        float *o = out + b * 32;
        uint16_t dbits = (uint16_t)(blk[0] | (blk[1] << 8));
        float d = oracle_f16_to_f32(dbits) * scale;
        if (ggml_type == OR_Q4_0) {
            /* low nibbles are elements 0..16, high nibbles 16..32, minus 8 */
            for (int j = 0; j < 16; j++) {
                uint8_t q = blk[2 + j];
                o[j] = (float)((int16_t)(q & 0x0f) - 8) * d;
                o[j + 16] = (float)((int16_t)(q >> 4) - 8) * d;
            }
        } else {
            for (int j = 0; j < 32; j++) o[j] = (float)(int8_t)blk[2 + j] * d;
        }
    }
    return 0;
}

/* rms_norm_rows (quant.rs:324-339), the scale-less norm of
 * Hparams::norm_embeddings (params.rs:374-379): per row, the squares of the
 * f32 values are summed in f64 in index order from 0 (Iterator::sum),
 * mean = sum / row_len, inv = (1 / sqrt(mean + f64(eps))) as f32, and every
 * value is multiplied by inv in f32. */
void oracle_rms_norm_rows(float *rows, int64_t n_rows, int64_t row_len, float eps) {
    for (int64_t r = 0; r < n_rows; r++) {
        float *row = rows + r * row_len;
        double sum = 0.0;
        for (int64_t i = 0; i < row_len; i++) sum += (double)row[i] * (double)row[i];
        const double mean = sum / (double)row_len;
        const float inv = (float)(1.0 / sqrt(mean + (double)eps));
        for (int64_t i = 0; i < row_len; i++) row[i] *= inv;
    }
}

typedef struct {
    const uint8_t *table;
    uint32_t type;
    int64_t hidden, row_bytes;
    const uint32_t *ids;
    float scale;
    int norm;
    float norm_eps;
    void *out;
    int dtype;
} embed_ctx;

static void embed_range(void *c, int64_t begin, int64_t end) {
    embed_ctx *e = (embed_ctx *)c;
    float *row = (float *)malloc(sizeof(float) * (size_t)e->hidden);
    for (int64_t t = begin; t < end; t++) {
        const uint8_t *src = e->table + (int64_t)e->ids[t] * e->row_bytes;
        oracle_dequant_row(e->type, src, e->row_bytes, e->scale, row, e->hidden);
        if (e->norm) oracle_rms_norm_rows(row, 1, e->hidden, e->norm_eps);
        if (e->dtype == OR_F16) {
            oracle_f32_to_f16_n(row, (uint16_t *)e->out + t * e->hidden, e->hidden);
        } else {
            memcpy((float *)e->out + t * e->hidden, row, sizeof(float) * (size_t)e->hidden);
        }
    }
    free(row);
}

/* TokenEmbedding::rows (quant.rs:391-411): bounds-check every id first
 * (the reference returns before writing anything useful), then dequantize
 * each row times `scale`. */
int oracle_embed_norm(const uint8_t *table, uint32_t ggml_type, int64_t vocab,
                      int64_t hidden, const uint32_t *ids, int64_t n_tok, float scale,
                      int norm, float norm_eps, void *out, int out_dtype, int nthreads,
                      int64_t *bad_index) {
    int64_t rb = oracle_row_bytes(ggml_type, hidden);
    if (rb < 0) return -1;
    for (int64_t t = 0; t < n_tok; t++) {
        if ((int64_t)ids[t] >= vocab) {
            if (bad_index) *bad_index = t;
            return -2;
        }
    }
    embed_ctx c = {table, ggml_type, hidden, rb, ids, scale, norm, norm_eps, out, out_dtype};
    parallel_rows(nthreads, n_tok, embed_range, &c);
    return 0;
}

int oracle_embed(const uint8_t *table, uint32_t ggml_type, int64_t vocab,
                 int64_t hidden, const uint32_t *ids, int64_t n_tok, float scale,
                 void *out, int out_dtype, int nthreads, int64_t *bad_index) {
    return oracle_embed_norm(table, ggml_type, vocab, hidden, ids, n_tok, scale, 0, 0.0f, out,
                             out_dtype, nthreads, bad_index);
}

/* ------------------------------------------------------------------ */
/* a5-a6: residual add + RMSNorm                                        */
/* ------------------------------------------------------------------ */

/* candle_nn::ops::rms_norm on one f32 row (cpu.rs:3652 -> candle-nn 0.11.1):
 * sum of squares in f32, index order; m = sqrt(sum/H + eps); y = v / m * w.
 * The GPU mirror of the same formula is gpu.rs:5883-5896. */
static void rms_row(const float *v, const float *w, float eps, int64_t H, float *y) {
    float sum2 = 0.0f;
    for (int64_t i = 0; i < H; i++) sum2 += v[i] * v[i];
    float m = sqrtf(sum2 / (float)H + eps);
    for (int64_t i = 0; i < H; i++) y[i] = w ? v[i] / m * w[i] : v[i] / m;
}

typedef struct {
    const void *x, *branch;
    const float *w, *w_post;
    float eps, post_eps, rs;
    int64_t H;
    void *x_out, *h_out;
    int dtype;
} norm_ctx;

static void norm_range(void *c, int64_t begin, int64_t end) {
    norm_ctx *n = (norm_ctx *)c;
    int64_t H = n->H;
    float *xv = (float *)malloc(sizeof(float) * (size_t)H * 3 + sizeof(uint16_t) * (size_t)H);
    float *bv = xv + H, *hv = bv + H;
    uint16_t *x16 = (uint16_t *)(hv + H);
    for (int64_t r = begin; r < end; r++) {
        load_row(n->x, r * H, H, n->dtype, xv);
        if (n->branch) {
            load_row(n->branch, r * H, H, n->dtype, bv);
            /* Gemma sandwich: post_attn_norm / post_ffw_norm on the branch
             * (cpu.rs:2675-2677, 2690-2692) */
            if (n->w_post) rms_row(bv, n->w_post, n->post_eps, H, bv);
            /* `scaled`: branch.affine(rs, 0) unless rs == 1 (cpu.rs:2661-2667) */
            if (n->rs != 1.0f)
                for (int64_t i = 0; i < H; i++) bv[i] = bv[i] * n->rs + 0.0f;
            for (int64_t i = 0; i < H; i++) xv[i] = xv[i] + bv[i];
        }
        /* the residual stream is held in the activation type: the norm reads
         * x' as stored */
        if (n->dtype == OR_F16) {
            oracle_f32_to_f16_n(xv, x16, H);
            oracle_f16_to_f32_n(x16, xv, H);
        }
        if (n->x_out) store_row(n->x_out, r * H, H, n->dtype, xv);
        rms_row(xv, n->w, n->eps, H, hv);
        store_row(n->h_out, r * H, H, n->dtype, hv);
    }
    free(xv);
}

void oracle_add_rmsnorm(const void *x, const void *branch, const float *w,
                        const float *w_post, float eps, float post_eps,
                        float residual_scale, int64_t rows, int64_t hidden,
                        void *x_out, void *h_out, int dtype, int nthreads) {
    norm_ctx c = {x, branch, w, w_post, eps, post_eps, residual_scale, hidden,
                  x_out, h_out, dtype};
    parallel_rows(nthreads, rows, norm_range, &c);
}

/* ------------------------------------------------------------------ */
/* a7: gated activation                                                 */
/* ------------------------------------------------------------------ */

/* candle's Tensor::silu / Tensor::gelu (tanh) scalar f32 forms, as the
 * reference restates them (gpu.rs:5899-5913, moe_kernel.rs:2340-2352). */
static inline float act_f32(float v, int act) {
    if (act == OR_SILU) return v / (1.0f + expf(-v));
    const float k = sqrtf(2.0f / 3.14159265358979323846f);
    return 0.5f * v * (1.0f + tanhf(k * v * (1.0f + 0.044715f * v * v)));
}

typedef struct {
    const void *gate, *up;
    int64_t gate_ld, up_ld, out_ld, ff;
    int act;
    float clamp;
    void *out;
    int dtype;
} glu_ctx;

static void glu_range(void *c, int64_t begin, int64_t end) {
    glu_ctx *g = (glu_ctx *)c;
    float *gb = (float *)malloc(sizeof(float) * (size_t)g->ff * 2);
    float *ub = gb + g->ff;
    for (int64_t r = begin; r < end; r++) {
        load_row(g->gate, r * g->gate_ld, g->ff, g->dtype, gb);
        load_row(g->up, r * g->up_ld, g->ff, g->dtype, ub);
        for (int64_t j = 0; j < g->ff; j++) {
            float gv = gb[j], uv = ub[j];
            if (g->clamp > 0.0f) { /* Glu::apply clamp (cpu.rs:364-368) */
                gv = gv < g->clamp ? gv : g->clamp;
                uv = uv > -g->clamp ? uv : -g->clamp;
                uv = uv < g->clamp ? uv : g->clamp;
            }
            gb[j] = act_f32(gv, g->act) * uv;
        }
        store_row(g->out, r * g->out_ld, g->ff, g->dtype, gb);
    }
    free(gb);
}

void oracle_glu(const void *gate, int64_t gate_ld, const void *up, int64_t up_ld,
                int64_t rows, int64_t ff, int act, float clamp, void *out,
                int64_t out_ld, int dtype, int nthreads) {
    glu_ctx c = {gate, up, gate_ld, up_ld, out_ld, ff, act, clamp, out, dtype};
    parallel_rows(nthreads, rows, glu_range, &c);
}

/* ------------------------------------------------------------------ */
/* a8-a9: RoPE tables and rotation                                      */
/* ------------------------------------------------------------------ */

/* ggml rope_yarn_corr_dim (rope.rs:86-90) */
static double corr_dim(int n_dims, int64_t n_ctx_orig, double n_rot, double base) {
    return (double)n_dims * log((double)n_ctx_orig / (n_rot * 2.0 * M_PI)) / (2.0 * log(base));
}

void oracle_rope_tables(int n_dims, double base, double freq_scale,
                        double yarn_ext_factor, double yarn_beta_fast,
                        double yarn_beta_slow, int64_t yarn_n_ctx_orig,
                        double attn_factor, const float *factors,
                        int64_t positions, float *cos_out, float *sin_out) {
    int half = n_dims / 2;
    double c0 = 0.0, c1 = 0.0;
    int yarn = yarn_ext_factor != 0.0;
    if (yarn) { /* Yarn::corr_dims (rope.rs:93-99) */
        double start = floor(corr_dim(n_dims, yarn_n_ctx_orig, yarn_beta_fast, base));
        double end = ceil(corr_dim(n_dims, yarn_n_ctx_orig, yarn_beta_slow, base));
        c0 = start > 0.0 ? start : 0.0;
        c1 = end < (double)(n_dims - 1) ? end : (double)(n_dims - 1);
    }
    for (int64_t pos = 0; pos < positions; pos++) {
        for (int i = 0; i < half; i++) {
            /* RopeSpec::angle (rope.rs:117-132) */
            double factor = factors ? (double)factors[i] : 1.0;
            int i0 = 2 * i;
            double extrap = (double)pos * pow(base, -(double)i0 / (double)n_dims) / factor;
            double interp = freq_scale * extrap;
            double theta, mscale;
            if (yarn) {
                double span = c1 - c0 > 0.001 ? c1 - c0 : 0.001;
                double t = ((double)(i0 / 2) - c0) / span;
                t = t < 0.0 ? 0.0 : (t > 1.0 ? 1.0 : t);
                double mix = (1.0 - t) * yarn_ext_factor;
                mscale = attn_factor * (1.0 + 0.1 * log(1.0 / freq_scale));
                theta = interp * (1.0 - mix) + extrap * mix;
            } else {
                theta = interp;
                mscale = attn_factor;
            }
            /* RopeSpec::tables (rope.rs:136-151): f64, then `as f32` */
            cos_out[pos * half + i] = (float)(cos(theta) * mscale);
            sin_out[pos * half + i] = (float)(sin(theta) * mscale);
        }
    }
}

typedef struct {
    void *x;
    int64_t ld;
    int heads, d, n_dims, kind;
    const float *cos_t, *sin_t;
    const int32_t *pos;
    const float *norm_w;
    float eps;
    int dtype;
    int full;   /* norm_w spans the whole row (heads * d): qk_norm_full */
} rope_ctx;

static void rope_range(void *c, int64_t begin, int64_t end) {
    rope_ctx *p = (rope_ctx *)c;
    int half = p->n_dims / 2;
    float *v = (float *)malloc(sizeof(float) * (size_t)p->d * 2);
    float *o = v + p->d;
    float *rowv = p->full ? (float *)malloc(sizeof(float) * (size_t)p->d * (size_t)p->heads) : NULL;
    for (int64_t r = begin; r < end; r++) {
        const float *cs = p->cos_t + (int64_t)p->pos[r] * half;
        const float *sn = p->sin_t + (int64_t)p->pos[r] * half;
        if (p->full) {
            /* the full-width QK-norm: rms over the whole projection row with
             * weights [heads * d], before the heads are split (cpu.rs:2838-2843,
             * 3042-3045) */
            int64_t w = (int64_t)p->heads * p->d;
            load_row(p->x, r * p->ld, w, p->dtype, rowv);
            if (p->norm_w) rms_row(rowv, p->norm_w, p->eps, w, rowv);
        }
        for (int h = 0; h < p->heads; h++) {
            int64_t at = r * p->ld + (int64_t)h * p->d;
            if (p->full) {
                memcpy(v, rowv + (int64_t)h * p->d, sizeof(float) * (size_t)p->d);
            } else {
                load_row(p->x, at, p->d, p->dtype, v);
                /* QK-norm per head: rms(q.reshape(1,t,nh,d), w[d]) (cpu.rs:2864) */
                if (p->norm_w) rms_row(v, p->norm_w, p->eps, p->d, v);
            }
            memcpy(o, v, sizeof(float) * (size_t)p->d);
            /* candle rope / rope_i = rotate_reference (rope.rs:158-171) */
            for (int i = 0; i < half; i++) {
                int a = p->kind == OR_ROPE_NEOX ? i : 2 * i;
                int b = p->kind == OR_ROPE_NEOX ? i + half : 2 * i + 1;
                o[a] = v[a] * cs[i] - v[b] * sn[i];
                o[b] = v[a] * sn[i] + v[b] * cs[i];
            }
            store_row(p->x, at, p->d, p->dtype, o);
        }
    }
    free(v);
    free(rowv);
}

void oracle_rope(void *x, int64_t ld, int64_t rows, int heads, int head_dim,
                 int n_dims, int kind, const float *cos_t, const float *sin_t,
                 const int32_t *positions, const float *norm_w, float eps,
                 int dtype, int nthreads) {
    rope_ctx c = {x, ld, heads, head_dim, n_dims, kind, cos_t, sin_t,
                  positions, norm_w, eps, dtype, 0};
    parallel_rows(nthreads, rows, rope_range, &c);
}

void oracle_rope_full(void *x, int64_t ld, int64_t rows, int heads, int head_dim,
                      int n_dims, int kind, const float *cos_t, const float *sin_t,
                      const int32_t *positions, const float *norm_w, float eps,
                      int dtype, int nthreads) {
    rope_ctx c = {x, ld, heads, head_dim, n_dims, kind, cos_t, sin_t,
                  positions, norm_w, eps, dtype, 1};
    parallel_rows(nthreads, rows, rope_range, &c);
}

/* ---- paged K/V pools (cpu/paged_attn.rs) ---- */

#define KV_BLOCK 16
#define KV_NO_BLOCK 0xffffffffu

/* check_range (paged_attn.rs:42-65) */
static int kv_range_ok(const uint32_t *table, int64_t table_len, int64_t lo, int64_t hi,
                       int64_t n_blocks) {
    if (lo >= hi) return 0;
    for (int64_t b = lo / KV_BLOCK; b <= (hi - 1) / KV_BLOCK; b++) {
        if (b >= table_len) return 0;
        uint32_t id = table[b];
        if (id == KV_NO_BLOCK || (int64_t)id >= n_blocks) return 0;
    }
    return 1;
}

/* row_offset (paged_attn.rs:33-38), in elements */
static int64_t kv_row_offset(const uint32_t *table, int64_t pos, int kvh, int n_kv, int d) {
    int64_t block = table[pos / KV_BLOCK];
    return ((block * n_kv + kvh) * KV_BLOCK + pos % KV_BLOCK) * (int64_t)d;
}

int oracle_store_rows(const uint32_t *table, int64_t table_len, int64_t start, int64_t rows,
                      const void *src, void *pool, int64_t n_blocks, int n_kv, int d,
                      int dtype) {
    size_t es = dtype == 1 ? 2 : 4;
    if (rows == 0) return 0;
    if (!kv_range_ok(table, table_len, start, start + rows, n_blocks)) return -1;
    for (int kvh = 0; kvh < n_kv; kvh++) {
        int64_t pos = start;
        while (pos < start + rows) {
            int64_t blk_end = (pos / KV_BLOCK + 1) * KV_BLOCK;
            int64_t end = start + rows < blk_end ? start + rows : blk_end;
            int64_t at = kv_row_offset(table, pos, kvh, n_kv, d);
            int64_t from = ((int64_t)kvh * rows + (pos - start)) * d;
            memcpy((char *)pool + at * es, (const char *)src + from * es, (size_t)((end - pos) * d) * es);
            pos = end;
        }
    }
    return 0;
}

int oracle_gather(const uint32_t *table, int64_t table_len, int64_t lo, int64_t hi,
                  const void *pool, void *out, int64_t n_blocks, int n_kv, int d, int dtype) {
    size_t es = dtype == 1 ? 2 : 4;
    if (!kv_range_ok(table, table_len, lo, hi, n_blocks)) return -1;
    char *o = (char *)out;
    for (int kvh = 0; kvh < n_kv; kvh++) {
        int64_t pos = lo;
        while (pos < hi) {
            int64_t blk_end = (pos / KV_BLOCK + 1) * KV_BLOCK;
            int64_t end = hi < blk_end ? hi : blk_end;
            int64_t at = kv_row_offset(table, pos, kvh, n_kv, d);
            size_t n = (size_t)((end - pos) * d) * es;
            memcpy(o, (const char *)pool + at * es, n);
            o += n;
            pos = end;
        }
    }
    return 0;
}

/* ---- paged attention (cpu/paged_attn.rs) ---- */

/* dot (paged_attn.rs:67-82): eight independent lanes, fixed order */
static float attn_dot(const float *a, const float *b, int n) {
    float lanes[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int n8 = n / 8 * 8;
    for (int j = 0; j < n8; j += 8)
        for (int i = 0; i < 8; i++) lanes[i] += a[j + i] * b[j + i];
    float sum = ((lanes[0] + lanes[4]) + (lanes[1] + lanes[5])) + ((lanes[2] + lanes[6]) + (lanes[3] + lanes[7]));
    for (int j = n8; j < n; j++) sum += a[j] * b[j];
    return sum;
}

typedef struct {
    const void *q;
    int n_head, n_kv, d;
    const uint32_t *tables;
    int64_t max_blocks;
    const int32_t *ranges;
    const void *pool_k, *pool_v;
    float scale;
    void *out;
    int dtype;
} attn_ctx;

static void attn_load(const void *src, int64_t at, int n, int dtype, float *dst) {
    if (dtype == 1) {
        const uint16_t *h = (const uint16_t *)src + at;
        for (int i = 0; i < n; i++) dst[i] = oracle_f16_to_f32(h[i]);
    } else {
        memcpy(dst, (const float *)src + at, sizeof(float) * (size_t)n);
    }
}

static void attn_range(void *c, int64_t begin, int64_t end) {
    attn_ctx *p = (attn_ctx *)c;
    int d = p->d, group = p->n_head / p->n_kv;
    float *qv = (float *)malloc(sizeof(float) * (size_t)d * 3);
    float *row = qv + d, *acc = qv + 2 * d;
    float scores[KV_BLOCK];
    for (int64_t job = begin; job < end; job++) {
        int64_t r = job / p->n_head;
        int head = (int)(job % p->n_head), kvh = head / group;
        const uint32_t *table = p->tables + r * p->max_blocks;
        int64_t lo = p->ranges[2 * r], hi = p->ranges[2 * r + 1];
        attn_load(p->q, job * d, d, p->dtype, qv);
        /* attend_head (paged_attn.rs:115-176) */
        for (int i = 0; i < d; i++) acc[i] = 0.0f;
        float mx = -INFINITY, sum = 0.0f;
        for (int64_t pos = lo; pos < hi;) {
            int64_t blk_end = (pos / KV_BLOCK + 1) * KV_BLOCK;
            int64_t e = hi < blk_end ? hi : blk_end;
            int n = (int)(e - pos);
            int64_t first = kv_row_offset(table, pos, kvh, p->n_kv, d);
            float block_max = -INFINITY;
            for (int j = 0; j < n; j++) {
                attn_load(p->pool_k, first + (int64_t)j * d, d, p->dtype, row);
                float sc = attn_dot(qv, row, d) * p->scale;
                scores[j] = sc;
                if (sc > block_max) block_max = sc;
            }
            if (block_max > mx) {
                float corr = expf(mx - block_max);
                sum *= corr;
                for (int i = 0; i < d; i++) acc[i] *= corr;
                mx = block_max;
            }
            for (int j = 0; j < n; j++) {
                float pr = expf(scores[j] - mx);
                sum += pr;
                attn_load(p->pool_v, first + (int64_t)j * d, d, p->dtype, row);
                for (int i = 0; i < d; i++) acc[i] += pr * row[i];
            }
            pos = e;
        }
        if (p->dtype == 1) {
            uint16_t *o = (uint16_t *)p->out + job * d;
            for (int i = 0; i < d; i++) o[i] = oracle_f32_to_f16(acc[i] / sum);
        } else {
            float *o = (float *)p->out + job * d;
            for (int i = 0; i < d; i++) o[i] = acc[i] / sum;
        }
    }
    free(qv);
}

int oracle_paged_attention(const void *q, int64_t rows, int n_head, int n_kv, int d,
                           const uint32_t *tables, int64_t max_blocks, const int32_t *ranges,
                           const void *pool_k, const void *pool_v, int64_t n_blocks, float scale,
                           void *out, int dtype, int nthreads) {
    if (n_kv <= 0 || n_head % n_kv != 0) return -1;
    for (int64_t r = 0; r < rows; r++) /* check_range, every row first */
        if (!kv_range_ok(tables + r * max_blocks, max_blocks, ranges[2 * r], ranges[2 * r + 1], n_blocks))
            return -1;
    attn_ctx c = {q, n_head, n_kv, d, tables, max_blocks, ranges, pool_k, pool_v, scale, out, dtype};
    parallel_rows(nthreads, rows * n_head, attn_range, &c);
    return 0;
}

/* ------------------------------------------------------------------ */
/* next, rank 3: the CPU engine's quantized matmul (QmmWeight)          */
/* ------------------------------------------------------------------ */

/* f32::round (ties away from zero), restating round_away (qmm.rs:1194-1201);
 * C's roundf has the same definition. */
static inline float qmm_round_away(float t) { return roundf(t); }

/* Rust's `f as i8`: saturating, NaN -> 0. */
static inline int8_t qmm_sat_i8(float t) {
    if (t != t) return 0;
    if (t >= 127.0f) return 127;
    if (t <= -128.0f) return -128;
    return (int8_t)t;
}

/* quantise_block (qmm.rs:1217-1240) for MIN_NONE. */
static float qmm_quantise_block(const float *src, int8_t *q) {
    float amax = 0.0f;
    for (int e = 0; e < 32; e++) amax = fmaxf(amax, fabsf(src[e])); /* max ignores NaN */
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    for (int e = 0; e < 32; e++) q[e] = qmm_sat_i8(qmm_round_away(src[e] * id));
    return oracle_f16_to_f32(oracle_f32_to_f16(d));
}

void oracle_q8_acts(const void *x, int64_t ld, int64_t m, int64_t k, int dtype,
                    int8_t *q, float *scales) {
    const int64_t nb = k / 32;
    float src[32];
    for (int64_t j = 0; j < m; j++)
        for (int64_t b = 0; b < nb; b++) {
            for (int e = 0; e < 32; e++) src[e] = load_el(x, j * ld + b * 32 + e, dtype);
            scales[j * nb + b] = qmm_quantise_block(src, q + j * k + b * 32);
        }
}

/* The block's f16 scale and its 32 quants as i16 in element order
 * (Legacy::scale / Legacy::halves: Q4_0 qmm.rs:240-263, Q8_0 qmm.rs:404-426). */
static float qmm_weight_block(uint32_t type, const uint8_t *blk, int16_t *w) {
    const float dw = oracle_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
    if (type == OR_Q4_0) {
        for (int i = 0; i < 16; i++) {
            w[i] = (int16_t)((blk[2 + i] & 0x0F) - 8);
            w[i + 16] = (int16_t)((blk[2 + i] >> 4) - 8);
        }
    } else {
        for (int i = 0; i < 32; i++) w[i] = (int16_t)(int8_t)blk[2 + i];
    }
    return dw;
}

/* hsum (qmm.rs:1345-1353): the fixed pairwise tree over the 16 lanes. */
static float qmm_hsum(const float *a) {
    float h[8];
    for (int i = 0; i < 8; i++) h[i] = a[i] + a[i + 8];
    return ((h[0] + h[4]) + (h[1] + h[5])) + ((h[2] + h[6]) + (h[3] + h[7]));
}

typedef struct {
    const uint8_t *w;
    uint32_t type;
    int64_t k, nb, row_bytes, m, rows;
    const int8_t *q;
    const float *xs;
    float *out;
} qmm_ctx;

/* Weight rows [begin, end) against every activation row: the scalar
 * definition of qmm/tests.rs:151-191 for a format without minima. */
static void qmm_range(void *c, int64_t begin, int64_t end) {
    qmm_ctx *g = (qmm_ctx *)c;
    const int bb = g->type == OR_Q4_0 ? 18 : 34;
    int16_t w[32];
    for (int64_t r = begin; r < end; r++) {
        for (int64_t j = 0; j < g->m; j++) {
            float lanes[16] = {0};
            for (int64_t b = 0; b < g->nb; b++) {
                const float dw = qmm_weight_block(g->type, g->w + r * g->row_bytes + b * bb, w);
                const int8_t *xq = g->q + j * g->k + b * 32;
                const float s = dw * g->xs[j * g->nb + b];
                for (int l = 0; l < 16; l++) {
                    const int32_t p = (int32_t)w[l] * xq[l] + (int32_t)w[l + 16] * xq[l + 16];
                    lanes[l] += (float)p * s;
                }
            }
            g->out[j * g->rows + r] = qmm_hsum(lanes);
        }
    }
}

int oracle_qmm(const uint8_t *w, uint32_t ggml_type, int64_t n, int64_t k,
               const void *x, int64_t ld, int64_t m, int64_t rows, float *out,
               int dtype, int nthreads) {
    if (ggml_type != OR_Q4_0 && ggml_type != OR_Q8_0) return -1;
    if (k <= 0 || k % 32 != 0 || rows <= 0 || rows > n || m < 0 || ld < k) return -1;
    if (m == 0) return 0;
    int8_t *q = (int8_t *)malloc((size_t)(m * k));
    float *xs = (float *)malloc(sizeof(float) * (size_t)(m * (k / 32)));
    if (!q || !xs) { free(q); free(xs); return -1; }
    oracle_q8_acts(x, ld, m, k, dtype, q, xs);
    qmm_ctx c = {w, ggml_type, k, k / 32, oracle_row_bytes(ggml_type, k), m, rows, q, xs, out};
    parallel_rows(nthreads, rows, qmm_range, &c);
    free(q);
    free(xs);
    return 0;
}

/* ------------------------------------------------------------------ */
/* next, rank 4: cap_logits and the sampler                            */
/* ------------------------------------------------------------------ */

void oracle_cap_logits(float *v, int64_t n, float logit_scale, float logit_mult, float softcap) {
    /* candle affine: mul and add are f64 converted to the element type */
    const float m1 = (float)(1.0 / (double)logit_scale);
    const float m2 = logit_mult;
    const float ci = softcap > 0.0f ? (float)(1.0 / (double)softcap) : 0.0f;
    for (int64_t i = 0; i < n; i++) {
        float x = v[i];
        if (logit_scale != 1.0f) x = x * m1 + 0.0f;
        if (logit_mult != 1.0f) x = x * m2 + 0.0f;
        if (softcap > 0.0f) x = tanhf(x * ci + 0.0f) * softcap + 0.0f;
        v[i] = x;
    }
}

uint32_t oracle_greedy(const float *logits, int64_t n) {
    int64_t best = 0;
    float bv = -INFINITY;
    for (int64_t i = 0; i < n; i++)
        if (logits[i] > bv) { best = i; bv = logits[i]; }
    return (uint32_t)best;
}

uint64_t oracle_splitmix64(uint64_t *state) {
    *state += 0x9E3779B97F4A7C15ull;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

float oracle_next_f32(uint64_t *state) {
    return (float)(oracle_splitmix64(state) >> 40) / 16777216.0f;
}

typedef struct { float v; uint32_t id; } cand_t;

/* f32::total_cmp as a signed 32-bit key (sampler.rs by_logit_desc). */
static int32_t total_key(float v) {
    int32_t b;
    memcpy(&b, &v, 4);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

/* by_logit_desc: descending total order, equal logits by ascending id. */
static int by_logit_desc(const void *pa, const void *pb) {
    const cand_t *a = (const cand_t *)pa, *b = (const cand_t *)pb;
    const int32_t ka = total_key(a->v), kb = total_key(b->v);
    if (ka != kb) return ka > kb ? -1 : 1;
    return a->id < b->id ? -1 : (a->id > b->id ? 1 : 0);
}

int64_t oracle_select_top_k(const float *logits, int64_t n, float temperature, int64_t k,
                            float *out_logits, uint32_t *out_ids) {
    cand_t *c = (cand_t *)malloc(sizeof(cand_t) * (size_t)(n > 0 ? n : 1));
    int64_t m = 0;
    for (int64_t i = 0; i < n; i++) {
        const float l = logits[i] / temperature;
        if (isfinite(l)) c[m++] = (cand_t){l, (uint32_t)i};
    }
    qsort(c, (size_t)m, sizeof(cand_t), by_logit_desc);
    const int64_t keep = m < k ? m : k;
    for (int64_t i = 0; i < keep; i++) {
        out_logits[i] = c[i].v;
        out_ids[i] = c[i].id;
    }
    free(c);
    return keep;
}

/* cut_top_p (sampler.rs:288-300) */
static int64_t cut_top_p(const cand_t *c, int64_t n, float top_p) {
    float cumulative = 0.0f;
    for (int64_t i = 0; i < n; i++) {
        cumulative += c[i].v;
        if (cumulative >= top_p) return i + 1;
    }
    return n;
}

/* softmax of candidates (logit -> exp(l - max)), then / sum, dropping zeros */
static int64_t softmax_retain(cand_t *c, int64_t n, float max) {
    float sum = 0.0f;
    for (int64_t i = 0; i < n; i++) {
        c[i].v = expf(c[i].v - max);
        sum += c[i].v;
    }
    int64_t m = 0;
    for (int64_t i = 0; i < n; i++) {
        const float p = c[i].v / sum;
        if (p > 0.0f) c[m++] = (cand_t){p, c[i].id};
    }
    return m;
}

uint32_t oracle_sample(float *logits, int64_t n, float temperature, int64_t top_k, float top_p,
                       uint64_t *rng) {
    if (temperature <= 0.0f || n <= 1) return oracle_greedy(logits, n);
    cand_t *c = (cand_t *)malloc(sizeof(cand_t) * (size_t)(n > 0 ? n : 1));
    int64_t m = 0;
    if (top_k > 0 && top_k < n) {
        /* select_top_k: scale in place, the k best finite of a full sort */
        for (int64_t i = 0; i < n; i++) logits[i] /= temperature;
        for (int64_t i = 0; i < n; i++)
            if (isfinite(logits[i])) c[m++] = (cand_t){logits[i], (uint32_t)i};
        qsort(c, (size_t)m, sizeof(cand_t), by_logit_desc);
        if (m > top_k) m = top_k;
        if (m == 0) {
            c[0] = (cand_t){1.0f, oracle_greedy(logits, n)};
            m = 1;
        } else {
            const float max = c[0].v;
            m = softmax_retain(c, m, max);
            if (m == 0) {
                c[0] = (cand_t){1.0f, oracle_greedy(logits, n)};
                m = 1;
            } else {
                m = cut_top_p(c, m, top_p);
            }
        }
    } else {
        /* the whole vocabulary (sampler.rs:191-252) */
        float max = -INFINITY;
        for (int64_t i = 0; i < n; i++) {
            logits[i] /= temperature;
            if (isfinite(logits[i])) {
                max = fmaxf(max, logits[i]);
                c[m++] = (cand_t){logits[i], (uint32_t)i};
            }
        }
        if (m == 0) {
            c[0] = (cand_t){1.0f, oracle_greedy(logits, n)};
            m = 1;
        } else if (top_p >= 1.0f) {
            m = softmax_retain(c, m, max);
            if (m == 0) {
                c[0] = (cand_t){1.0f, oracle_greedy(logits, n)};
                m = 1;
            }
        } else {
            /* sum over every candidate in vocabulary order; the nucleus is
             * the shortest sorted prefix, widened from 256 fourfold while its
             * mass is below top_p (NUCLEUS_FIRST, :154) */
            float sum = 0.0f;
            for (int64_t i = 0; i < m; i++) sum += expf(c[i].v - max);
            qsort(c, (size_t)m, sizeof(cand_t), by_logit_desc);
            int64_t w = m < 256 ? m : 256;
            for (;;) {
                float mass = 0.0f;
                for (int64_t i = 0; i < w; i++) mass += expf(c[i].v - max);
                mass /= sum;
                if (mass >= top_p || w >= m) break;
                w = w * 4 < m ? w * 4 : m;
            }
            int64_t k2 = 0;
            for (int64_t i = 0; i < w; i++) {
                const float p = expf(c[i].v - max) / sum;
                if (p > 0.0f) c[k2++] = (cand_t){p, c[i].id};
            }
            if (k2 == 0) {
                c[0] = (cand_t){1.0f, oracle_greedy(logits, n)};
                m = 1;
            } else {
                m = cut_top_p(c, k2, top_p);
            }
        }
    }
    float total = 0.0f;
    for (int64_t i = 0; i < m; i++) total += c[i].v;
    const float target = oracle_next_f32(rng) * total;
    float acc = 0.0f;
    uint32_t out = c[m - 1].id;
    for (int64_t i = 0; i < m; i++) {
        acc += c[i].v;
        if (target < acc) { out = c[i].id; break; }
    }
    free(c);
    return out;
}
