/*
 * q3k_oracle.c -- CPU restatement of the reference runtime's non-GEMM layer
 * arithmetic.  TEST INFRASTRUCTURE ONLY (see q3k_oracle.h): only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * Build: gcc -O2 -ffp-contract=off (see oracle/Makefile).  Contraction is
 * off so that every fp32 product and sum below is rounded exactly where the
 * source says; fmaf() marks the one place where the reference kernel is
 * assumed to be contracted by nvcc (rms_norm.cu:89, "sum += v * v").
 *
 * Functions follow, and cite, the reference files under src/ops/.  CUDA's
 * rsqrtf and expf cannot be restated bit for bit; the primary result uses
 * the correctly rounded 1.0f/sqrtf(.) and (float)exp((double).), and the
 * per-element band [lo, hi] covers the difference (q3k_oracle.h).
 */
#include "q3k_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---- bf16 ------------------------------------------------------------- */

uint16_t q3o_bf16_from_f32(float x)
{
    uint32_t b;
    memcpy(&b, &x, sizeof b);
    if ((b & 0x7fffffffu) > 0x7f800000u)
        return (uint16_t)((b >> 16) | 0x0040u);
    b += 0x7fffu + ((b >> 16) & 1u);
    return (uint16_t)(b >> 16);
}

float q3o_f32_from_bf16(uint16_t v)
{
    const uint32_t b = (uint32_t)v << 16;
    float f;
    memcpy(&f, &b, sizeof f);
    return f;
}

#define BF q3o_bf16_from_f32
#define FB q3o_f32_from_bf16

static int is_nan_bf(uint16_t v) { return (v & 0x7fffu) > 0x7f80u; }

static int32_t ord_bf(uint16_t v)
{
    return (v & 0x8000u) ? -(int32_t)(v & 0x7fffu) : (int32_t)v;
}

int32_t q3o_ulp_distance(uint16_t a, uint16_t b)
{
    const int na = is_nan_bf(a), nb = is_nan_bf(b);
    if (na || nb)
        return (na && nb) ? 0 : INT32_MAX;
    const int32_t d = ord_bf(a) - ord_bf(b);
    return d < 0 ? -d : d;
}

static uint16_t min_bf(uint16_t a, uint16_t b) { return ord_bf(a) <= ord_bf(b) ? a : b; }
static uint16_t max_bf(uint16_t a, uint16_t b) { return ord_bf(a) >= ord_bf(b) ? a : b; }

/* Relative half-widths of the fp32 noise bands.  2^-21 is 4..8 fp32 ulps:
 * CUDA rsqrtf and expf are documented at <= 2 ulp, IEEE divide/sqrt add
 * 0.5 ulp each, and any pairwise-ish fp32 sum of <= 8192 squares stays well
 * inside the rest. */
double q3o_band_rel_inv(void) { return ldexp(1.0, -21); }
double q3o_band_rel_silu(void) { return ldexp(1.0, -21); }

/* Spacing of fp32 values at |v| (as a double). */
static double ulp_f32(double v)
{
    const float a = (float)fabs(v);
    if (a == 0.0f)
        return ldexp(1.0, -149);
    if (isinf(a))
        return INFINITY;
    return (double)nextafterf(a, INFINITY) - (double)a;
}

/* bf16 of the fp32 rounding of a double (monotone in v). */
static uint16_t bf_of_double(double v) { return BF((float)v); }

/* ---- tiny parallel-for ----------------------------------------------- */

typedef void (*range_fn)(void *ctx, int64_t begin, int64_t end);

/* A pool of worker threads kept for the life of the process, grown to the
 * largest thread count asked for: a call hands part i of [0, n) to worker i
 * (the caller takes part 0) and returns when every part is done.  Calls are
 * serialised (one job at a time). */
#define POOL_MAX 256
static pthread_mutex_t pool_call = PTHREAD_MUTEX_INITIALIZER;
static pthread_mutex_t pool_lock = PTHREAD_MUTEX_INITIALIZER;
static pthread_cond_t pool_go = PTHREAD_COND_INITIALIZER;
static pthread_cond_t pool_done = PTHREAD_COND_INITIALIZER;
static int pool_workers = 0;          /* workers started: parts 1 .. pool_workers */
static unsigned long pool_job = 0;    /* generation of the current job */
static int pool_parts = 0;            /* parts of the current job */
static int pool_pending = 0;          /* parts 1 .. pool_parts - 1 not yet finished */
static range_fn pool_fn;
static void *pool_ctx;
static int64_t pool_n;

static void *pool_worker(void *arg)
{
    const int part = (int)(intptr_t)arg;
    unsigned long seen = 0;
    pthread_mutex_lock(&pool_lock);
    for (;;)
    {
        while (pool_job == seen)
            pthread_cond_wait(&pool_go, &pool_lock);
        seen = pool_job;
        if (part >= pool_parts)
            continue;
        const range_fn fn = pool_fn;
        void *ctx = pool_ctx;
        const int64_t b = pool_n * part / pool_parts, e = pool_n * (part + 1) / pool_parts;
        pthread_mutex_unlock(&pool_lock);
        fn(ctx, b, e);
        pthread_mutex_lock(&pool_lock);
        if (--pool_pending == 0)
            pthread_cond_signal(&pool_done);
    }
    return NULL;
}

static void parallel_for(int64_t n, int nthreads, range_fn fn, void *ctx)
{
    if (nthreads <= 1 || n < 2)
    {
        fn(ctx, 0, n);
        return;
    }
    if (nthreads > POOL_MAX)
        nthreads = POOL_MAX;
    if ((int64_t)nthreads > n)
        nthreads = (int)n;
    pthread_mutex_lock(&pool_call);
    pthread_mutex_lock(&pool_lock);
    while (pool_workers < nthreads - 1)
    {
        pthread_t t;
        if (pthread_create(&t, NULL, pool_worker, (void *)(intptr_t)(pool_workers + 1)) != 0)
            break;
        pthread_detach(t);
        ++pool_workers;
    }
    const int parts = pool_workers + 1 < nthreads ? pool_workers + 1 : nthreads;
    pool_fn = fn;
    pool_ctx = ctx;
    pool_n = n;
    pool_parts = parts;
    pool_pending = parts - 1;
    ++pool_job;
    pthread_cond_broadcast(&pool_go);
    pthread_mutex_unlock(&pool_lock);
    fn(ctx, 0, n / parts);
    pthread_mutex_lock(&pool_lock);
    while (pool_pending > 0)
        pthread_cond_wait(&pool_done, &pool_lock);
    pthread_mutex_unlock(&pool_lock);
    pthread_mutex_unlock(&pool_call);
}

/* ---- embedding: src/ops/embedding.cu:29-54 ----------------------------- */

struct emb_ctx
{
    const int32_t *ids;
    const uint16_t *table;
    int64_t V, H;
    uint16_t *out;
};

static void emb_range(void *p, int64_t b, int64_t e)
{
    const struct emb_ctx *c = (const struct emb_ctx *)p;
    for (int64_t t = b; t < e; ++t)
    {
        const int32_t id = c->ids[t];
        uint16_t *dst = c->out + t * c->H;
        if (id < 0 || (int64_t)id >= c->V)
            memset(dst, 0, (size_t)c->H * sizeof(uint16_t)); /* __float2bfloat16(0.0F) */
        else
            memcpy(dst, c->table + (int64_t)id * c->H, (size_t)c->H * sizeof(uint16_t));
    }
}

void q3o_embedding(const int32_t *ids, int64_t T, const uint16_t *table, int64_t V, int64_t H,
                   uint16_t *out, int nthreads)
{
    struct emb_ctx c = {ids, table, V, H, out};
    parallel_for(T, nthreads, emb_range, &c);
}

/* ---- add: src/ops/elementwise.cu:28-35 --------------------------------- */

struct add_ctx
{
    uint16_t *d;
    const uint16_t *s;
};

static void add_range(void *p, int64_t b, int64_t e)
{
    const struct add_ctx *c = (const struct add_ctx *)p;
    for (int64_t i = b; i < e; ++i)
        c->d[i] = BF(FB(c->d[i]) + FB(c->s[i]));
}

void q3o_add_inplace(uint16_t *d, const uint16_t *s, int64_t n, int nthreads)
{
    struct add_ctx c = {d, s};
    parallel_for(n, nthreads, add_range, &c);
}

/* ---- rms_norm: src/ops/rms_norm.cu:22-67, 82-121 ----------------------- */

/* Lane 0 of __shfl_down_sync tree over 32 lanes (rms_norm.cu:22-30). */
static float warp_tree(const float *in)
{
    float v[32];
    memcpy(v, in, sizeof v);
    for (int off = 16; off > 0; off >>= 1)
        for (int i = 0; i < off; ++i)
            v[i] = v[i] + v[i + off];
    return v[0];
}

/* Sum of squares in the reference kernel's order: 256 threads, thread j
 * accumulates columns j, j+256, ... (rms_norm.cu:85-90, contracted), then
 * the per-warp trees and the tree over the 8 warp partials (:32-67). */
static float ref_sum_squares(const uint16_t *x, int64_t n)
{
    float part[256];
    for (int j = 0; j < 256; ++j)
    {
        float p = 0.0f;
        for (int64_t c = j; c < n; c += 256)
        {
            const float v = FB(x[c]);
            p = fmaf(v, v, p);
        }
        part[j] = p;
    }
    float block[32];
    memset(block, 0, sizeof block);
    for (int w = 0; w < 8; ++w)
        block[w] = warp_tree(part + 32 * w);
    return warp_tree(block);
}

/* Normalise one row.  x_row holds the (already rounded) bf16 inputs. */
static void rms_row(const uint16_t *x, const uint16_t *w, int64_t n, float eps, uint16_t *y, uint16_t *lo,
                    uint16_t *hi)
{
    const float sum = ref_sum_squares(x, n);
    const float mean = sum / (float)n;
    const float inv = 1.0f / sqrtf(mean + eps); /* stands in for rsqrtf (rms_norm.cu:98) */

    for (int64_t c = 0; c < n; ++c)
    {
        const uint16_t nrm = BF(FB(x[c]) * inv);
        y[c] = BF(FB(nrm) * FB(w[c]));
    }
    if (lo == NULL || hi == NULL)
        return;

    double exact = 0.0;
    for (int64_t c = 0; c < n; ++c)
    {
        const double v = FB(x[c]);
        exact += v * v;
    }
    const double inv_exact = 1.0 / sqrt(exact / (double)n + (double)eps);
    const double rel = q3o_band_rel_inv();
    const double a = fmin((double)inv, inv_exact) * (1.0 - rel);
    const double b = fmax((double)inv, inv_exact) * (1.0 + rel);
    for (int64_t c = 0; c < n; ++c)
    {
        const double xv = FB(x[c]);
        const uint16_t na = bf_of_double(xv * a), nb = bf_of_double(xv * b);
        const uint16_t nprim = BF(FB(x[c]) * inv);
        const uint16_t nlo = min_bf(min_bf(na, nb), nprim), nhi = max_bf(max_bf(na, nb), nprim);
        const float wv = FB(w[c]);
        const uint16_t ya = BF(FB(nlo) * wv), yb = BF(FB(nhi) * wv);
        lo[c] = min_bf(min_bf(ya, yb), y[c]);
        hi[c] = max_bf(max_bf(ya, yb), y[c]);
    }
}

struct rms_ctx
{
    uint16_t *h;
    const uint16_t *x, *d, *w;
    int64_t n;
    float eps;
    uint16_t *y, *lo, *hi;
};

static void rms_range(void *p, int64_t b, int64_t e)
{
    const struct rms_ctx *c = (const struct rms_ctx *)p;
    for (int64_t r = b; r < e; ++r)
    {
        const int64_t off = r * c->n;
        const uint16_t *src = c->x + off;
        if (c->d != NULL)
        {
            /* residual add first (elementwise.cu:34), the norm reads the rounded h */
            for (int64_t i = 0; i < c->n; ++i)
                c->h[off + i] = BF(FB(c->h[off + i]) + FB(c->d[off + i]));
            src = c->h + off;
        }
        rms_row(src, c->w, c->n, c->eps, c->y + off, c->lo ? c->lo + off : NULL, c->hi ? c->hi + off : NULL);
    }
}

void q3o_rms_norm(const uint16_t *x, const uint16_t *w, int64_t rows, int64_t N, float eps, uint16_t *y,
                  uint16_t *lo, uint16_t *hi, int nthreads)
{
    struct rms_ctx c = {NULL, x, NULL, w, N, eps, y, lo, hi};
    parallel_for(rows, nthreads, rms_range, &c);
}

/* The reference test's CPU loop (tests/unit/rms_norm_cuda_test.cpp:174-244):
 * the fp32 sum of squares in column order, 1 / sqrt(sum / N + eps), then
 * the kernel's two roundings. */
struct rms_seq_ctx
{
    const uint16_t *x, *w;
    int64_t n;
    float eps;
    uint16_t *y;
};

static void rms_seq_range(void *p, int64_t b, int64_t e)
{
    const struct rms_seq_ctx *c = (const struct rms_seq_ctx *)p;
    for (int64_t r = b; r < e; ++r)
    {
        const uint16_t *x = c->x + r * c->n;
        uint16_t *y = c->y + r * c->n;
        float sum = 0.0f;
        for (int64_t i = 0; i < c->n; ++i)
        {
            const float v = FB(x[i]);
            sum += v * v;
        }
        const float inv = 1.0f / sqrtf(sum / (float)c->n + c->eps);
        for (int64_t i = 0; i < c->n; ++i)
            y[i] = BF(FB(BF(FB(x[i]) * inv)) * FB(c->w[i]));
    }
}

void q3o_rms_norm_test_order(const uint16_t *x, const uint16_t *w, int64_t rows, int64_t N, float eps, uint16_t *y,
                             int nthreads)
{
    struct rms_seq_ctx c = {x, w, N, eps, y};
    parallel_for(rows, nthreads, rms_seq_range, &c);
}

void q3o_add_rms_norm(uint16_t *h, const uint16_t *d, const uint16_t *w, int64_t rows, int64_t N, float eps,
                      uint16_t *y, uint16_t *lo, uint16_t *hi, int nthreads)
{
    struct rms_ctx c = {h, h, d, w, N, eps, y, lo, hi};
    parallel_for(rows, nthreads, rms_range, &c);
}

/* ---- silu(gate) * up: src/ops/elementwise.cu:45-66 ----------------------- */

struct silu_ctx
{
    const uint16_t *g, *u;
    uint16_t *out, *lo, *hi;
};

static void silu_range(void *p, int64_t b, int64_t e)
{
    const struct silu_ctx *c = (const struct silu_ctx *)p;
    const double rel = q3o_band_rel_silu();
    for (int64_t i = b; i < e; ++i)
    {
        const float g = FB(c->g[i]);
        const float u = FB(c->u[i]);
        const float ex = (float)exp(-(double)g); /* stands in for expf (elementwise.cu:51) */
        const float den = 1.0f + ex;
        const float s = g / den;
        const uint16_t n = BF(s);
        c->out[i] = BF(FB(n) * u);
        if (c->lo == NULL || c->hi == NULL)
            continue;
        double sx;
        const double E = exp(-(double)g);
        if (isinf((float)E))
            sx = (double)g / INFINITY; /* fp32 exp overflows: silu is a signed zero */
        else
            sx = (double)g / (1.0 + E);
        const uint16_t na = bf_of_double(sx * (1.0 - rel)), nb = bf_of_double(sx * (1.0 + rel));
        const uint16_t nlo = min_bf(min_bf(na, nb), n), nhi = max_bf(max_bf(na, nb), n);
        const uint16_t oa = BF(FB(nlo) * u), ob = BF(FB(nhi) * u);
        c->lo[i] = min_bf(min_bf(oa, ob), c->out[i]);
        c->hi[i] = max_bf(max_bf(oa, ob), c->out[i]);
    }
}

void q3o_silu_mul(const uint16_t *g, const uint16_t *u, int64_t n, uint16_t *out, uint16_t *lo, uint16_t *hi,
                  int nthreads)
{
    struct silu_ctx c = {g, u, out, lo, hi};
    parallel_for(n, nthreads, silu_range, &c);
}

/* ---- rope: src/ops/rope.cu:38-85, 267-296 -------------------------------- */

int q3o_build_rope_cache(int64_t P, int32_t D, float theta, float *cache)
{
    if (P <= 0 || D <= 0 || (D % 2) != 0 || !(theta > 0.0f) || isinf(theta) || cache == NULL)
        return -1;
    const int64_t half = D / 2;
    double *inv = (double *)malloc((size_t)half * sizeof(double));
    if (inv == NULL)
        return -1;
    for (int64_t i = 0; i < half; ++i)
        inv[i] = pow((double)theta, -((2.0 * (double)i) / (double)D));
    for (int64_t p = 0; p < P; ++p)
        for (int64_t i = 0; i < half; ++i)
        {
            const double angle = (double)p * inv[i];
            cache[(p * half + i) * 2] = (float)cos(angle);
            cache[(p * half + i) * 2 + 1] = (float)sin(angle);
        }
    free(inv);
    return 0;
}

/* Interval [lo, hi] of bf16 values for v1 * c + v2 * s2 with v1 in
 * [a_lo, a_hi], v2 in [b_lo, b_hi] (fp32 values), widened by the rounding
 * of the two products and the sum in any contraction order (1.5 ulp of the
 * larger product). */
static void rot_band(float a_lo, float a_hi, float c, float b_lo, float b_hi, float s2, uint16_t prim,
                     uint16_t *lo, uint16_t *hi)
{
    const double p1 = (double)a_lo * c, p2 = (double)a_hi * c;
    const double q1 = (double)b_lo * s2, q2 = (double)b_hi * s2;
    const double mn = fmin(p1, p2) + fmin(q1, q2);
    const double mx = fmax(p1, p2) + fmax(q1, q2);
    const double big = fmax(fmax(fabs(p1), fabs(p2)), fmax(fabs(q1), fabs(q2)));
    const double err = 1.5 * ulp_f32(big);
    *lo = min_bf(bf_of_double(mn - err), prim);
    *hi = max_bf(bf_of_double(mx + err), prim);
}

struct rope_ctx
{
    uint16_t *x;
    const uint16_t *w; /* non-NULL: fused norm first */
    int64_t S;
    int32_t heads, D;
    float eps;
    const float *cache;
    int64_t P, start;
    const int32_t *positions;
    uint16_t *lo, *hi;
};

static void rope_range(void *p, int64_t b, int64_t e)
{
    const struct rope_ctx *c = (const struct rope_ctx *)p;
    const int64_t D = c->D, half = D / 2;
    uint16_t *nrm = (uint16_t *)malloc((size_t)D * 3 * sizeof(uint16_t));
    if (nrm == NULL)
        abort();
    uint16_t *nlo = nrm + D, *nhi = nrm + 2 * D;
    for (int64_t t = b; t < e; ++t)
    {
        const int64_t pos = c->positions ? (int64_t)c->positions[t] : c->start + t % c->S;
        for (int32_t hd = 0; hd < c->heads; ++hd)
        {
            uint16_t *head = c->x + (t * c->heads + hd) * D;
            uint16_t *hlo = c->lo ? c->lo + (t * c->heads + hd) * D : NULL;
            uint16_t *hhi = c->hi ? c->hi + (t * c->heads + hd) * D : NULL;
            if (pos < 0 || pos >= c->P)
            {
                for (int64_t i = 0; i < D; ++i)
                {
                    head[i] = 0x7fc0;
                    if (hlo)
                        hlo[i] = hhi[i] = 0x7fc0;
                }
                continue;
            }
            if (c->w != NULL)
            {
                /* self_attention.cpp:147-149: rms_norm over the head, two roundings */
                rms_row(head, c->w, D, c->eps, nrm, hlo ? nlo : NULL, hlo ? nhi : NULL);
                memcpy(head, nrm, (size_t)D * sizeof(uint16_t));
            }
            else if (hlo)
            {
                memcpy(nlo, head, (size_t)D * sizeof(uint16_t));
                memcpy(nhi, head, (size_t)D * sizeof(uint16_t));
            }
            for (int64_t i = 0; i < half; ++i)
            {
                const float cs = c->cache[(pos * half + i) * 2];
                const float sn = c->cache[(pos * half + i) * 2 + 1];
                const float x1 = FB(head[i]), x2 = FB(head[i + half]);
                const float a = x1 * cs, bb = x2 * sn, ee = x2 * cs, ff = x1 * sn;
                const uint16_t o1 = BF(a - bb), o2 = BF(ee + ff);
                if (hlo)
                {
                    rot_band(FB(nlo[i]), FB(nhi[i]), cs, FB(nlo[i + half]), FB(nhi[i + half]), -sn, o1, &hlo[i],
                             &hhi[i]);
                    rot_band(FB(nlo[i + half]), FB(nhi[i + half]), cs, FB(nlo[i]), FB(nhi[i]), sn, o2,
                             &hlo[i + half], &hhi[i + half]);
                }
                head[i] = o1;
                head[i + half] = o2;
            }
        }
    }
    free(nrm);
}

static int rope_common(uint16_t *x, const uint16_t *w, int64_t B, int64_t S, int32_t heads, int32_t D, float eps,
                       const float *cache, int64_t P, int64_t start, const int32_t *positions, uint16_t *lo,
                       uint16_t *hi, int nthreads)
{
    if (B < 0 || S < 0 || heads <= 0 || D <= 0 || D % 2 != 0 || P <= 0)
        return -1;
    if (positions == NULL && (start < 0 || start > P || S > P - start))
        return -1;
    if ((lo == NULL) != (hi == NULL))
        return -1;
    struct rope_ctx c = {x, w, S, heads, D, eps, cache, P, start, positions, lo, hi};
    parallel_for(B * S, nthreads, rope_range, &c);
    return 0;
}

int q3o_rope(uint16_t *x, int64_t B, int64_t S, int32_t heads, int32_t D, const float *cache, int64_t P,
             int64_t start, const int32_t *positions, uint16_t *lo, uint16_t *hi, int nthreads)
{
    return rope_common(x, NULL, B, S, heads, D, 0.0f, cache, P, start, positions, lo, hi, nthreads);
}

int q3o_qk_norm_rope(uint16_t *x, const uint16_t *w, int64_t B, int64_t S, int32_t heads, int32_t D, float eps,
                     const float *cache, int64_t P, int64_t start, const int32_t *positions, uint16_t *lo,
                     uint16_t *hi, int nthreads)
{
    if (w == NULL)
        return -1;
    return rope_common(x, w, B, S, heads, D, eps, cache, P, start, positions, lo, hi, nthreads);
}

/* ---- comparison ----------------------------------------------------------- */

void q3o_compare_band(const uint16_t *got, const uint16_t *primary, const uint16_t *lo, const uint16_t *hi,
                      int64_t n, int64_t *stats)
{
    for (int i = 0; i < 8; ++i)
        stats[i] = 0;
    stats[0] = n;
    stats[2] = -1;
    for (int64_t i = 0; i < n; ++i)
    {
        const uint16_t l = lo ? lo[i] : primary[i];
        const uint16_t h = hi ? hi[i] : primary[i];
        const int32_t dist = q3o_ulp_distance(got[i], primary[i]);
        if (dist == 0)
            stats[4]++;
        else if (dist == 1)
            stats[5]++;
        else if (dist == 2)
            stats[6]++;
        else
            stats[7]++;
        if (ord_bf(l) != ord_bf(h))
            stats[3]++;
        int ok;
        if (is_nan_bf(got[i]) || is_nan_bf(primary[i]))
            ok = is_nan_bf(got[i]) && is_nan_bf(primary[i]);
        else
            ok = ord_bf(got[i]) >= ord_bf(l) - 1 && ord_bf(got[i]) <= ord_bf(h) + 1;
        if (!ok)
        {
            if (stats[2] < 0)
                stats[2] = i;
            stats[1]++;
        }
    }
}

/* ---- KV-cache append: src/model/kv_cache.cpp:147-185 ------------------- */

void q3o_kv_append(const void *k, const void *v, void *kc, void *vc, int64_t B, int64_t S, int64_t row_bytes,
                   int64_t seq_cap, int64_t start)
{
    const int64_t width = S * row_bytes;          /* source pitch = copy width */
    const int64_t dst_pitch = seq_cap * row_bytes; /* one batch row of the cache */
    for (int64_t b = 0; b < B; ++b)
    {
        memcpy((char *)kc + b * dst_pitch + start * row_bytes, (const char *)k + b * width, (size_t)width);
        memcpy((char *)vc + b * dst_pitch + start * row_bytes, (const char *)v + b * width, (size_t)width);
    }
}

/* ---- grouped-query attention: src/ops/gqa_attention.cu:20-155 ------------ */

struct attn_ctx
{
    const uint16_t *q, *k, *v;
    int64_t S;
    int32_t Hq, Hkv, D;
    int64_t cached, start;
    const int64_t *ks, *vs;
    const int64_t *rows;
    uint16_t *out, *lo, *hi;
    float scale;
};

/* The kernel's dot product: thread t < D holds q_t * k_t, threads D..255
 * hold 0, then the shared-memory tree with offsets 128, 64, ..., 1
 * (gqa_attention.cu:75-104). */
static float attn_ref_dot(const float *qv, const uint16_t *kp, int64_t kd, int D)
{
    float r[256];
    for (int t = 0; t < 256; ++t)
        r[t] = t < D ? qv[t] * FB(kp[t * kd]) : 0.0f;
    for (int off = 128; off > 0; off /= 2)
        for (int t = 0; t < off; ++t)
            r[t] += r[t + off];
    return r[0];
}

/* Half-width of the band on one output: a first-order bound on what fp32
 * arithmetic can change, relative to the value in double.  Terms: the dot
 * product, summed by the reference as a binary tree of depth 8 (256 slots)
 * and by a matrix-core kernel in at most 16 rounded steps (chunks of exact
 * products), hence gamma_16 on sum |q k| (a sum of depth d errs by at most
 * gamma_d sum |x|); the
 * scale product, the subtraction and exp of each weight (4 u for expf, 2 u on
 * the argument), one exp-and-multiply per later rescale of the running
 * maximum, and the accumulation of numerator and denominator over the visible
 * keys, bounded probabilistically (Higham and Mary, SIAM J. Sci. Comput. 41
 * (2019) A2815: lambda * sqrt(n) * u with lambda = 8, failing with probability
 * below 2 n exp(-32) per output) because a worst-case
 * n * u for n in the thousands would exceed a bf16 ulp without any
 * implementation coming near it.  The divide adds 2 u. */
static void attn_band(const struct attn_ctx *c, const float *qv, const uint16_t *kb, const uint16_t *vb,
                      int64_t vis, double *work, const float *prim, uint16_t *lo, uint16_t *hi)
{
    const double u = ldexp(1.0, -24);
    const int D = c->D;
    const double gD = 16.0 * u / (1.0 - 16.0 * u);
    const double gL = 8.0 * sqrt(3.0 * (double)vis) * u;
    const double e_exp = 4.0 * u;
    double *sd = work, *ad = work + vis, *rj = work + 2 * vis;
    double M = -INFINITY;
    for (int64_t j = 0; j < vis; ++j)
    {
        const uint16_t *kp = kb + j * c->ks[1];
        double s = 0.0, a = 0.0;
        for (int t = 0; t < D; ++t)
        {
            const double p = (double)qv[t] * (double)FB(kp[t * c->ks[3]]);
            s += p;
            a += fabs(p);
        }
        sd[j] = s * (double)c->scale;
        ad[j] = a * (double)c->scale;
        if (sd[j] > M)
            M = sd[j];
    }
    /* rescales after key j: strict increases of the running maximum */
    double run = -INFINITY, later = 0.0;
    for (int64_t j = 0; j < vis; ++j)
    {
        rj[j] = (j > 0 && sd[j] > run) ? 1.0 : 0.0;
        if (sd[j] > run)
            run = sd[j];
    }
    for (int64_t j = vis - 1; j >= 0; --j)
    {
        const double inc = rj[j];
        rj[j] = later + 1.0;
        later += inc;
    }
    double den = 0.0, eden = 0.0;
    for (int64_t j = 0; j < vis; ++j)
    {
        const double w = exp(sd[j] - M);
        const double e = gD * ad[j] + u * fabs(sd[j]) + 2.0 * u * fabs(sd[j] - M) + e_exp + rj[j] * (e_exp + 2.0 * u);
        den += w;
        eden += w * e;
        sd[j] = w; /* reuse: weight */
        ad[j] = e; /* reuse: relative error of the weight */
    }
    eden += gL * den;
    for (int t = 0; t < D; ++t)
    {
        double num = 0.0, absn = 0.0, enum_ = 0.0;
        for (int64_t j = 0; j < vis; ++j)
        {
            const double x = (double)FB(vb[j * c->vs[1] + t * c->vs[3]]);
            num += sd[j] * x;
            absn += sd[j] * fabs(x);
            enum_ += sd[j] * fabs(x) * ad[j];
        }
        enum_ += gL * absn;
        const double o = num / den;
        const double E = (enum_ + fabs(o) * eden) / den + 2.0 * u * fabs(o);
        const uint16_t p = BF(prim[t]);
        lo[t] = min_bf(bf_of_double(o - E), p);
        hi[t] = max_bf(bf_of_double(o + E), p);
    }
}

static void attn_range(void *p, int64_t b, int64_t e)
{
    const struct attn_ctx *c = (const struct attn_ctx *)p;
    const int D = c->D;
    const int32_t G = c->Hq / c->Hkv;
    double *work = (double *)malloc(sizeof(double) * 3 * (size_t)(c->cached > 0 ? c->cached : 1));
    float qv[256], acc[256], res[256];
    for (int64_t i = b; i < e; ++i)
    {
        const int64_t row = c->rows ? c->rows[i] : i;
        const int32_t h = (int32_t)(row % c->Hq);
        const int64_t bs = row / c->Hq;
        const int64_t s = bs % c->S, bi = bs / c->S;
        const int32_t kvh = h / G;
        const int64_t vis = c->start + s + 1;
        const uint16_t *kb = c->k + bi * c->ks[0] + kvh * c->ks[2];
        const uint16_t *vb = c->v + bi * c->vs[0] + kvh * c->vs[2];
        for (int t = 0; t < D; ++t)
        {
            qv[t] = FB(c->q[row * D + t]);
            acc[t] = 0.0f;
        }
        float m = -INFINITY, l = 0.0f;
        for (int64_t j = 0; j < vis; ++j)
        {
            const float score = attn_ref_dot(qv, kb + j * c->ks[1], c->ks[3], D) * c->scale;
            const float nm = fmaxf(m, score);
            const float ow = (float)exp((double)(m - nm)); /* stands in for expf (:111) */
            const float nw = (float)exp((double)(score - nm));
            l = fmaf(l, ow, nw);
            const uint16_t *vp = vb + j * c->vs[1];
            for (int t = 0; t < D; ++t)
                acc[t] = fmaf(FB(vp[t * c->vs[3]]), nw, acc[t] * ow);
            m = nm;
        }
        for (int t = 0; t < D; ++t)
        {
            res[t] = acc[t] / l;
            c->out[i * D + t] = BF(res[t]);
        }
        if (c->lo && c->hi)
            attn_band(c, qv, kb, vb, vis, work, res, c->lo + i * D, c->hi + i * D);
    }
    free(work);
}

int q3o_gqa_attention(const uint16_t *q, const uint16_t *k, const uint16_t *v, int64_t B, int64_t S, int32_t Hq,
                      int32_t Hkv, int32_t D, int64_t cached, int64_t start, const int64_t *k_strides,
                      const int64_t *v_strides, const int64_t *rows, int64_t nrows, uint16_t *out, uint16_t *lo,
                      uint16_t *hi, int nthreads)
{
    if (B <= 0 || S <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || D <= 0 || D > 256 || start < 0 ||
        start + S != cached)
        return -1;
    const int64_t total = B * S * Hq;
    for (int64_t i = 0; rows && i < nrows; ++i)
        if (rows[i] < 0 || rows[i] >= total)
            return -1;
    struct attn_ctx c = {q, k, v, S, Hq, Hkv, D, cached, start, k_strides, v_strides, rows, out, lo, hi,
                         1.0f / sqrtf((float)D)}; /* host scale, gqa_attention.cu:322 */
    parallel_for(rows ? nrows : total, nthreads, attn_range, &c);
    return 0;
}

/* ---- argmax over the last dimension: src/ops/argmax.cu:28-100 ----------- */

void q3o_argmax(const uint16_t *x, int64_t rows, int64_t row_stride, int64_t search_size, int32_t *out)
{
    for (int64_t r = 0; r < rows; ++r)
    {
        float best = -INFINITY;
        int32_t best_index = 2147483647; /* kInvalidIndex (:25) */
        for (int64_t c = 0; c < search_size; ++c)
        {
            float v = FB(x[r * row_stride + c]);
            if (v != v)
                v = -INFINITY; /* NaN counts as -inf (:54-58) */
            if (v > best || (v == best && (int32_t)c < best_index))
            {
                best = v;
                best_index = (int32_t)c;
            }
        }
        out[r] = best_index;
    }
}

/* ---- sampling: src/generation/sampler.cpp:17-34, 134-265 ---------------- */

struct q3o_cand
{
    double score;
    int32_t id;
};

/* candidate_is_better (:21-27) as a qsort order: higher score first, then
 * the smaller id */
static int cand_order(const void *pa, const void *pb)
{
    const struct q3o_cand *a = (const struct q3o_cand *)pa, *b = (const struct q3o_cand *)pb;
    if (a->score != b->score)
        return a->score > b->score ? -1 : 1;
    return a->id < b->id ? -1 : (a->id > b->id ? 1 : 0);
}

/* Temperature scores of row[0 .. n-1] and the reference's top-k rule: keep
 * every candidate whose score is >= the k-th best (:160-190); returns the
 * kept count, candidates sorted best first.  -1 for a non-finite logit. */
static int64_t topk_sorted(const uint16_t *row, int64_t n, double temperature, int32_t top_k, struct q3o_cand *c)
{
    for (int64_t t = 0; t < n; ++t)
    {
        const float logit = FB(row[t]);
        if (!isfinite(logit))
            return -1;
        c[t].score = (double)logit / temperature;
        c[t].id = (int32_t)t;
    }
    qsort(c, (size_t)n, sizeof *c, cand_order);
    int64_t kept = n;
    if (top_k > 0 && (int64_t)top_k < n)
    {
        const double kth = c[top_k - 1].score;
        kept = top_k;
        while (kept < n && c[kept].score >= kth)
            ++kept;
    }
    return kept;
}

int64_t q3o_topk_set(const uint16_t *row, int64_t n, int32_t k, int32_t *ids)
{
    struct q3o_cand *c = (struct q3o_cand *)malloc(sizeof *c * (size_t)n);
    const int64_t kept = topk_sorted(row, n, 1.0, k, c);
    for (int64_t i = 0; i < kept; ++i)
        ids[i] = c[i].id;
    free(c);
    return kept;
}

int32_t q3o_sample_row(const uint16_t *row, int64_t n, float temperature, int32_t top_k, float top_p, double u)
{
    struct q3o_cand *c = (struct q3o_cand *)malloc(sizeof *c * (size_t)n);
    double *w = (double *)malloc(sizeof *w * (size_t)n);
    int32_t token = -1;
    const int64_t kept = topk_sorted(row, n, (double)temperature, top_k, c);
    if (kept > 0)
    {
        /* stable softmax (:198-215) */
        const double maximum = c[0].score;
        double total = 0.0;
        for (int64_t i = 0; i < kept; ++i)
        {
            w[i] = exp(c[i].score - maximum);
            total += w[i];
        }
        /* top-p: first prefix whose weight reaches top_p * total (:221-238) */
        const double threshold = (double)top_p * total;
        int64_t retained = kept;
        double retained_weight = 0.0;
        for (int64_t i = 0; i < kept; ++i)
        {
            retained_weight += w[i];
            if (retained_weight >= threshold)
            {
                retained = i + 1;
                break;
            }
        }
        /* draw (:244-262) */
        const double r = u * retained_weight;
        double cumulative = 0.0;
        token = c[retained - 1].id;
        for (int64_t i = 0; i < retained; ++i)
        {
            cumulative += w[i];
            if (r < cumulative)
            {
                token = c[i].id;
                break;
            }
        }
    }
    free(w);
    free(c);
    return token;
}
