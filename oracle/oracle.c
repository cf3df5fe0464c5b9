/*
 * oracle.c -- CPU oracle for the XCD-domain kernels. TEST INFRASTRUCTURE ONLY: loaded by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg; never by the product.
 *
 * Pinning (what checks each function against something other than itself) is listed in
 * tests/test_oracle.py; a function without such a check is marked "parity unpinned" here.
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------------------ */
/* threading helper                                                                      */
/* ------------------------------------------------------------------------------------ */
typedef void (*range_fn)(void *ctx, int64_t begin, int64_t end);
typedef struct {
    range_fn fn;
    void *ctx;
    int64_t b, e;
} range_job;

static void *range_tramp(void *p) {
    range_job *j = (range_job *)p;
    j->fn(j->ctx, j->b, j->e);
    return NULL;
}

static void parallel_range(int64_t n, int nthreads, range_fn fn, void *ctx) {
    if (nthreads <= 1 || n < 2) {
        fn(ctx, 0, n);
        return;
    }
    if (nthreads > 256) nthreads = 256;
    pthread_t th[256];
    range_job jobs[256];
    int64_t per = (n + nthreads - 1) / nthreads;
    int started = 0;
    for (int t = 0; t < nthreads; ++t) {
        int64_t b = (int64_t)t * per, e = b + per < n ? b + per : n;
        if (b >= e) break;
        jobs[t].fn = fn;
        jobs[t].ctx = ctx;
        jobs[t].b = b;
        jobs[t].e = e;
        if (pthread_create(&th[t], NULL, range_tramp, &jobs[t]) != 0) {
            fn(ctx, b, e);
            continue;
        }
        started = t + 1;
    }
    for (int t = 0; t < started; ++t) pthread_join(th[t], NULL);
}

/* ------------------------------------------------------------------------------------ */
/* generators                                                                            */
/* ------------------------------------------------------------------------------------ */

/* splitmix64 (Steele, Lea, Flood 2014): state += 0x9e3779b97f4a7c15, then the variant-13
 * output mix. Output number `index` of the stream whose initial state is `seed`. */
uint64_t ora_splitmix64(uint64_t seed, uint64_t index) {
    uint64_t z = seed + (index + 1) * 0x9e3779b97f4a7c15ULL;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

/* GEMV.cu:56-63 (also HIST.cu:333-338, HASH.cu:29-36). */
uint32_t ora_mix32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

/* binary64 -> binary16, round to nearest even, by integer manipulation of the bits. */
uint16_t ora_f64_to_f16(double d) {
    uint64_t b;
    memcpy(&b, &d, 8);
    uint16_t sign = (uint16_t)((b >> 48) & 0x8000u);
    uint64_t E = (b >> 52) & 0x7ffu;
    uint64_t m = b & 0xfffffffffffffULL;
    if (E == 0x7ff) return (uint16_t)(sign | (m ? 0x7e00u : 0x7c00u));
    if (E == 0) return sign; /* zero or binary64 subnormal: far below 2^-25 */
    int64_t e = (int64_t)E - 1023;
    if (e > 15) return (uint16_t)(sign | 0x7c00u);
    if (e >= -14) {
        uint64_t hm = m >> 42, rem = m & ((1ULL << 42) - 1), half = 1ULL << 41;
        uint32_t r = (uint32_t)(((uint64_t)(e + 15) << 10) | hm);
        if (rem > half || (rem == half && (hm & 1))) ++r; /* carries into exponent / inf */
        return (uint16_t)(sign | r);
    }
    uint64_t M = (1ULL << 52) | m;
    int64_t shift = 42 + (-14 - e);
    if (shift >= 54) return sign;
    uint64_t q = M >> shift, rem = M & ((1ULL << shift) - 1), half = 1ULL << (shift - 1);
    if (rem > half || (rem == half && (q & 1))) ++q;
    return (uint16_t)(sign | (uint16_t)q);
}

double ora_f16_to_f64(uint16_t h) {
    int s = (h >> 15) & 1, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    double v;
    if (e == 0) v = ldexp((double)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexp((double)(m | 0x400), e - 25);
    return s ? -v : v;
}

void ora_gen_uniform_f32(float *out, size_t n, uint64_t seed) {
    for (size_t i = 0; i < n; ++i) {
        int32_t k = (int32_t)(ora_splitmix64(seed, i) >> 40) - (1 << 23);
        out[i] = (float)ldexp((double)k, -23);
    }
}

void ora_gen_normal_f16(uint16_t *out, size_t n, double mean, double stddev, uint64_t seed) {
    const double two_pi = 2.0 * 3.14159265358979323846264338327950288;
    for (size_t j = 0; 2 * j < n; ++j) {
        double u1 = ldexp((double)((ora_splitmix64(seed, 2 * j) >> 11) + 1), -53);
        double u2 = ldexp((double)(ora_splitmix64(seed, 2 * j + 1) >> 11), -53);
        double r = sqrt(-2.0 * log(u1));
        out[2 * j] = ora_f64_to_f16(mean + stddev * (r * cos(two_pi * u2)));
        if (2 * j + 1 < n) out[2 * j + 1] = ora_f64_to_f16(mean + stddev * (r * sin(two_pi * u2)));
    }
}

/* ------------------------------------------------------------------------------------ */
/* GEMV                                                                                  */
/* ------------------------------------------------------------------------------------ */
typedef struct {
    const void *A, *x;
    float *yf;
    double *yd, *yabs;
    int64_t K;
} gemv_ctx;

/* GEMV.cu:383-390: sum += a[k] * x[k] in float, k ascending. */
static void gemv_seq_rows(void *p, int64_t b, int64_t e) {
    gemv_ctx *c = (gemv_ctx *)p;
    const float *A = (const float *)c->A, *x = (const float *)c->x;
    for (int64_t r = b; r < e; ++r) {
        float sum = 0.0f;
        const float *a = A + r * c->K;
        for (int64_t k = 0; k < c->K; ++k) {
            float prod = a[k] * x[k];
            sum = sum + prod;
        }
        c->yf[r] = sum;
    }
}

static void gemv_f64_rows(void *p, int64_t b, int64_t e) {
    gemv_ctx *c = (gemv_ctx *)p;
    const float *A = (const float *)c->A, *x = (const float *)c->x;
    for (int64_t r = b; r < e; ++r) {
        double s = 0.0, sa = 0.0;
        const float *a = A + r * c->K;
        for (int64_t k = 0; k < c->K; ++k) {
            double t = (double)a[k] * (double)x[k];
            s += t;
            sa += fabs(t);
        }
        c->yd[r] = s;
        if (c->yabs) c->yabs[r] = sa;
    }
}

static void gemv_f16_rows(void *p, int64_t b, int64_t e) {
    gemv_ctx *c = (gemv_ctx *)p;
    const uint16_t *W = (const uint16_t *)c->A, *x = (const uint16_t *)c->x;
    double *xd = (double *)malloc(sizeof(double) * (size_t)c->K);
    for (int64_t k = 0; k < c->K; ++k) xd[k] = ora_f16_to_f64(x[k]);
    for (int64_t r = b; r < e; ++r) {
        double s = 0.0, sa = 0.0;
        const uint16_t *w = W + r * c->K;
        for (int64_t k = 0; k < c->K; ++k) {
            double t = ora_f16_to_f64(w[k]) * xd[k];
            s += t;
            sa += fabs(t);
        }
        c->yd[r] = s;
        if (c->yabs) c->yabs[r] = sa;
    }
    free(xd);
}

void ora_gemv_f32_seq(const float *A, const float *x, float *y, int64_t M, int64_t K, int nthreads) {
    gemv_ctx c = {A, x, y, NULL, NULL, K};
    parallel_range(M, nthreads, gemv_seq_rows, &c);
}

void ora_gemv_f32_f64(const float *A, const float *x, double *y, double *yabs, int64_t M, int64_t K,
                      int nthreads) {
    gemv_ctx c = {A, x, NULL, y, yabs, K};
    parallel_range(M, nthreads, gemv_f64_rows, &c);
}

void ora_gemv_f16_f64(const uint16_t *W, const uint16_t *x, double *y, double *yabs, int64_t M,
                      int64_t K, int nthreads) {
    gemv_ctx c = {W, x, NULL, y, yabs, K};
    parallel_range(M, nthreads, gemv_f16_rows, &c);
}

/* ------------------------------------------------------------------------------------ */
/* histogram                                                                             */
/* ------------------------------------------------------------------------------------ */
void ora_zipf_thresholds(uint64_t *t, uint32_t num_bins, double s) {
    /* H = sum_{r=1..N} r^-s, accumulated in rank order in double. */
    double H = 0.0;
    for (uint32_t r = 1; r <= num_bins; ++r) H += pow((double)r, -s);
    double cum = 0.0;
    for (uint32_t k = 0; k < num_bins; ++k) {
        cum += pow((double)(k + 1), -s);
        double f = cum / H;
        if (k + 1 == num_bins || f >= 1.0) t[k] = UINT64_MAX;
        else t[k] = (uint64_t)ldexp(f, 64);
    }
}

uint32_t ora_zipf_scramble(uint32_t rank, uint32_t num_bins) {
    /* affine bijection on [0, 2^m): (rank + 1) * 0x9E3779B1 mod 2^m; identity otherwise */
    if (num_bins == 0 || (num_bins & (num_bins - 1))) return rank;
    return (uint32_t)(((uint64_t)(rank + 1) * 0x9E3779B1ULL) & (num_bins - 1));
}

uint32_t ora_zipf_key_at(const uint64_t *t, uint32_t num_bins, uint64_t seed, int scramble, uint64_t index) {
    uint64_t u = ora_splitmix64(seed, index);
    uint32_t k = 0;
    while (k + 1 < num_bins && !(u < t[k])) ++k; /* linear search: independent of the device's bisection */
    return scramble ? ora_zipf_scramble(k, num_bins) : k;
}

void ora_gen_zipf_keys(uint32_t *keys, size_t n, const uint64_t *t, uint32_t num_bins, uint64_t seed,
                       int scramble) {
    for (size_t i = 0; i < n; ++i) keys[i] = ora_zipf_key_at(t, num_bins, seed, scramble, i);
}

typedef struct {
    const uint32_t *keys;
    uint32_t num_bins;
    uint32_t **priv;
    uint64_t *counted;
    int64_t per;
} hist_ctx;

static void hist_part(void *p, int64_t b, int64_t e) {
    hist_ctx *c = (hist_ctx *)p;
    int64_t t = b / c->per;
    uint32_t *h = c->priv[t];
    uint64_t cnt = 0;
    for (int64_t i = b; i < e; ++i) {
        uint32_t k = c->keys[i];
        if (k < c->num_bins) {
            h[k]++;
            cnt++;
        }
    }
    c->counted[t] = cnt;
}

/* HIST.cu:279-288: serial counting loop; with nthreads > 1, private histograms then a sum. */
uint64_t ora_histogram(const uint32_t *keys, size_t n, uint32_t *counts, uint32_t num_bins, int nthreads) {
    memset(counts, 0, sizeof(uint32_t) * num_bins);
    if (nthreads <= 1 || n < 4096) {
        uint64_t cnt = 0;
        for (size_t i = 0; i < n; ++i)
            if (keys[i] < num_bins) {
                counts[keys[i]]++;
                cnt++;
            }
        return cnt;
    }
    if (nthreads > 256) nthreads = 256;
    uint32_t *priv[256];
    uint64_t counted[256];
    for (int t = 0; t < nthreads; ++t) {
        priv[t] = (uint32_t *)calloc(num_bins, sizeof(uint32_t));
        counted[t] = 0;
    }
    hist_ctx c = {keys, num_bins, priv, counted, (int64_t)((n + nthreads - 1) / nthreads)};
    parallel_range((int64_t)n, nthreads, hist_part, &c);
    uint64_t total = 0;
    for (int t = 0; t < nthreads; ++t) {
        for (uint32_t k = 0; k < num_bins; ++k) counts[k] += priv[t][k];
        total += counted[t];
        free(priv[t]);
    }
    return total;
}

/* The reference's own histogram data and loop (HIST.cu:331-340, 279-288): words[i] =
 * mix32((uint32_t)i ^ seed) (seed 0 in the reference), and every byte of every word
 * counted into 256 bins. */
void ora_gen_mix32_words(uint32_t *out, size_t n, uint32_t seed) {
    for (size_t i = 0; i < n; ++i) out[i] = ora_mix32((uint32_t)i ^ seed);
}

typedef struct {
    const uint32_t *w;
    uint32_t (*priv)[256];
    int64_t per;
} h256_ctx;

static void h256_part(void *p, int64_t b, int64_t e) {
    h256_ctx *c = (h256_ctx *)p;
    uint32_t *h = c->priv[b / c->per];
    for (int64_t i = b; i < e; ++i) {
        const uint32_t w = c->w[i];
        h[w & 0xffu]++;
        h[(w >> 8) & 0xffu]++;
        h[(w >> 16) & 0xffu]++;
        h[w >> 24]++;
    }
}

void ora_hist256_bytes(const uint32_t *words, size_t n, uint32_t *counts, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    uint32_t(*priv)[256] = (uint32_t(*)[256])calloc((size_t)nthreads, sizeof(*priv));
    h256_ctx c = {words, priv, (int64_t)((n + nthreads - 1) / nthreads)};
    if (c.per < 1) c.per = 1;
    parallel_range((int64_t)n, nthreads, h256_part, &c);
    memset(counts, 0, 256 * sizeof(uint32_t));
    for (int t = 0; t < nthreads; ++t)
        for (int k = 0; k < 256; ++k) counts[k] += priv[t][k];
    free(priv);
}

/* GEMV init_data (GEMV.cu:118-139): h = mix32((uint32_t)i ^ seed); the default inputs are
 * (float)(h & 0xff) / 255.0f - 0.5f, the INTEGER_FLOAT_INPUTS ones (int)(h % modulus) - offset. */
void ora_gen_mix32_f32(float *out, size_t n, uint32_t seed, uint32_t modulus, int32_t offset) {
    for (size_t i = 0; i < n; ++i) {
        const uint32_t h = ora_mix32((uint32_t)i ^ seed);
        if (modulus) {
            out[i] = (float)((int32_t)(h % modulus) - offset);
        } else {
            const float q = (float)(h & 0xffu) / 255.0f;
            out[i] = q - 0.5f;
        }
    }
}

/* ------------------------------------------------------------------------------------ */
/* hash table                                                                            */
/* ------------------------------------------------------------------------------------ */
#define ORA_EMPTY 0xFFFFFFFFFFFFFFFFULL

uint64_t ora_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

void ora_hash_kv(uint64_t *keys, uint64_t *vals, uint64_t n, uint64_t seed) {
    for (uint64_t i = 0; i < n; ++i) {
        keys[i] = ora_splitmix64(seed, i);
        if (vals) vals[i] = ora_splitmix64(seed ^ 0x5bd1e9955bd1e995ULL, i);
    }
}

void ora_hash_queries(uint64_t *q, uint64_t n, uint64_t n_keys, uint64_t seed, uint64_t qseed) {
    for (uint64_t j = 0; j < n; ++j) {
        uint64_t idx = (j & 1) ? n_keys + (j >> 1) : ora_splitmix64(qseed, j) % n_keys;
        q[j] = ora_splitmix64(seed, idx);
    }
}

static uint64_t probe_limit(uint64_t slots) { return slots < 65536 ? slots : 65536; }

/* HASH.cu:232-241: slot = hash & mask; advance while occupied; store. Here the stored key
 * may already be the same key (then only the value changes). */
uint64_t ora_hash_build(uint64_t *tkeys, uint64_t *tvals, uint64_t slots, const uint64_t *keys,
                        const uint64_t *vals, uint64_t n) {
    uint64_t mask = slots - 1, failed = 0, lim = probe_limit(slots);
    for (uint64_t s = 0; s < slots; ++s) {
        tkeys[s] = ORA_EMPTY;
        tvals[s] = 0;
    }
    for (uint64_t i = 0; i < n; ++i) {
        uint64_t k = keys[i];
        if (k == ORA_EMPTY) continue;
        uint64_t s = ora_mix64(k) & mask, step;
        for (step = 0; step < lim; ++step) {
            if (tkeys[s] == ORA_EMPTY || tkeys[s] == k) {
                tkeys[s] = k;
                tvals[s] = vals[i];
                break;
            }
            s = (s + 1) & mask;
        }
        if (step == lim) failed++;
    }
    return failed;
}

typedef struct {
    const uint64_t *tkeys, *tvals, *q;
    uint64_t mask, lim;
    uint64_t *vals_out;
    uint8_t *found_out;
} lookup_ctx;

/* HASH.cu:46-64: probe until the key or EMPTY. */
static void lookup_range(void *p, int64_t b, int64_t e) {
    lookup_ctx *c = (lookup_ctx *)p;
    for (int64_t i = b; i < e; ++i) {
        uint64_t q = c->q[i], v = 0;
        uint8_t f = 0;
        if (q != ORA_EMPTY) {
            uint64_t s = ora_mix64(q) & c->mask;
            for (uint64_t step = 0; step < c->lim; ++step) {
                if (c->tkeys[s] == q) {
                    v = c->tvals[s];
                    f = 1;
                    break;
                }
                if (c->tkeys[s] == ORA_EMPTY) break;
                s = (s + 1) & c->mask;
            }
        }
        c->vals_out[i] = v;
        c->found_out[i] = f;
    }
}

void ora_hash_lookup(const uint64_t *tkeys, const uint64_t *tvals, uint64_t slots, const uint64_t *q,
                     uint64_t n, uint64_t *vals_out, uint8_t *found_out, int nthreads) {
    lookup_ctx c = {tkeys, tvals, q, slots - 1, probe_limit(slots), vals_out, found_out};
    parallel_range((int64_t)n, nthreads, lookup_range, &c);
}

/* ------------------------------------------------------------------------------------ */
/* R-MAT and BFS                                                                         */
/* ------------------------------------------------------------------------------------ */
void ora_rmat_edge(int scale, double a, double b, double c, uint64_t seed, uint64_t e, int32_t *u, int32_t *v) {
    uint32_t ta = (uint32_t)floor(a * 4294967296.0), tab = (uint32_t)floor((a + b) * 4294967296.0),
             tabc = (uint32_t)floor((a + b + c) * 4294967296.0);
    uint64_t words = (uint64_t)(scale + 1) / 2;
    uint32_t uu = 0, vv = 0;
    for (int l = 0; l < scale; ++l) {
        uint64_t w = ora_splitmix64(seed, e * words + (uint64_t)(l / 2));
        uint32_t r = (l & 1) ? (uint32_t)(w >> 32) : (uint32_t)w;
        int row = r >= tab;            /* quadrants c, d */
        int colb = (r >= ta && r < tab) || r >= tabc; /* quadrants b, d */
        uu = (uu << 1) | (uint32_t)row;
        vv = (vv << 1) | (uint32_t)colb;
    }
    *u = (int32_t)uu;
    *v = (int32_t)vv;
}

static int cmp_i32(const void *x, const void *y) {
    int32_t a = *(const int32_t *)x, b = *(const int32_t *)y;
    return (a > b) - (a < b);
}

int64_t ora_rmat_csr(int scale, int edge_factor, double a, double b, double c, uint64_t seed, int32_t *rowptr,
                     int32_t *col) {
    int64_t V = (int64_t)1 << scale, E = (int64_t)edge_factor * V;
    int64_t *deg = (int64_t *)calloc((size_t)V + 1, sizeof(int64_t));
    int32_t *eu = (int32_t *)malloc(sizeof(int32_t) * (size_t)E), *ev = (int32_t *)malloc(sizeof(int32_t) * (size_t)E);
    for (int64_t e = 0; e < E; ++e) {
        ora_rmat_edge(scale, a, b, c, seed, (uint64_t)e, &eu[e], &ev[e]);
        if (eu[e] != ev[e]) {
            deg[eu[e]]++;
            deg[ev[e]]++;
        }
    }
    int64_t *off = (int64_t *)malloc(sizeof(int64_t) * ((size_t)V + 1)), *fill = (int64_t *)calloc((size_t)V, sizeof(int64_t));
    off[0] = 0;
    for (int64_t i = 0; i < V; ++i) off[i + 1] = off[i] + deg[i];
    int32_t *tmp = (int32_t *)malloc(sizeof(int32_t) * (size_t)(off[V] > 0 ? off[V] : 1));
    for (int64_t e = 0; e < E; ++e)
        if (eu[e] != ev[e]) {
            tmp[off[eu[e]] + fill[eu[e]]++] = ev[e];
            tmp[off[ev[e]] + fill[ev[e]]++] = eu[e];
        }
    int64_t n = 0;
    rowptr[0] = 0;
    for (int64_t v = 0; v < V; ++v) {
        int64_t len = off[v + 1] - off[v];
        qsort(tmp + off[v], (size_t)len, sizeof(int32_t), cmp_i32);
        for (int64_t j = 0; j < len; ++j)
            if (j == 0 || tmp[off[v] + j] != tmp[off[v] + j - 1]) col[n++] = tmp[off[v] + j];
        rowptr[v + 1] = (int32_t)n;
    }
    free(deg);
    free(eu);
    free(ev);
    free(off);
    free(fill);
    free(tmp);
    return n;
}

/* Textbook BFS with a FIFO queue; level = depth of first discovery (bfs.cu:240, :30). */
int64_t ora_bfs(const int32_t *rowptr, const int32_t *col, int32_t V, int32_t src, uint32_t *level) {
    for (int32_t v = 0; v < V; ++v) level[v] = 0xffffffffu;
    int32_t *q = (int32_t *)malloc(sizeof(int32_t) * (size_t)V);
    int64_t head = 0, tail = 0;
    level[src] = 0;
    q[tail++] = src;
    while (head < tail) {
        int32_t u = q[head++];
        for (int32_t e = rowptr[u]; e < rowptr[u + 1]; ++e) {
            int32_t v = col[e];
            if (level[v] == 0xffffffffu) {
                level[v] = level[u] + 1;
                q[tail++] = v;
            }
        }
    }
    free(q);
    return tail;
}

/* Multi-source fixed-depth BFS (bfs.cu:151-174 seeds, 215-252 levels, 449-491 fixed loop):
 * every source at 0, then max_depth top-down levels; returns the number of reached vertices. */
int64_t ora_bfs_multi(const int32_t *rowptr, const int32_t *col, int32_t V, const int32_t *src, int32_t nsrc,
                      int32_t max_depth, uint32_t *level) {
    for (int32_t v = 0; v < V; ++v) level[v] = 0xffffffffu;
    int32_t *q = (int32_t *)malloc(sizeof(int32_t) * (size_t)(V > 0 ? V : 1));
    int64_t head = 0, tail = 0;
    for (int32_t i = 0; i < nsrc; ++i)
        if (level[src[i]] != 0u) {
            level[src[i]] = 0u;
            q[tail++] = src[i];
        }
    while (head < tail) {
        const int32_t u = q[head++];
        if ((int32_t)level[u] >= max_depth) continue; /* the last level is not expanded */
        for (int32_t e = rowptr[u]; e < rowptr[u + 1]; ++e) {
            const int32_t v = col[e];
            if (level[v] == 0xffffffffu) {
                level[v] = level[u] + 1;
                q[tail++] = v;
            }
        }
    }
    free(q);
    return tail;
}

/* The reference's graph (bfs.cu:354-409, see xdom.h's xd_bfs_ref_graph for the rule): row
 * side = home of col_addr + 4 v degree, level side = home of level_addr + 4 v, home = bit 13
 * of the address ^ attr[page] (or the parity of address & mask without a map). Returns 0, or
 * -1 when a hot pool cannot be filled. */
static uint8_t ora_side(uint64_t addr, uint64_t base, const uint8_t *attr, uint64_t mask) {
    if (attr) return (uint8_t)(((addr >> 13) & 1u) ^ attr[(addr >> 21) - (base >> 21)]);
    return (uint8_t)(__builtin_popcountll(addr & mask) & 1);
}

int ora_bfs_ref_graph(int32_t V, int32_t degree, int32_t nsrc, int32_t dst_local_pct, int32_t H, uint64_t seed,
                      uint64_t col_addr, const uint8_t *col_home, uint64_t level_addr, const uint8_t *level_home,
                      uint64_t mask, int32_t *rowptr, int32_t *col, uint8_t *work_side, int32_t *src) {
    int32_t *hot0 = (int32_t *)malloc(sizeof(int32_t) * (size_t)H), *hot1 = (int32_t *)malloc(sizeof(int32_t) * (size_t)H);
    uint8_t *vside = (uint8_t *)malloc((size_t)V), *dside = (uint8_t *)malloc((size_t)V);
    int32_t n0 = 0, n1 = 0;
    for (int32_t v = 0; v < V; ++v) {
        const uint8_t rs = ora_side(col_addr + (uint64_t)v * (uint64_t)degree * 4u, col_addr, col_home, mask);
        const uint8_t ds = ora_side(level_addr + (uint64_t)v * 4u, level_addr, level_home, mask);
        vside[v] = rs;
        if (rs != ds) continue;
        if (rs == 0 && n0 < H) hot0[n0++] = v;
        if (rs == 1 && n1 < H) hot1[n1++] = v;
    }
    int rc = 0;
    if (n0 < H || n1 < H) {
        rc = -1;
    } else {
        for (int32_t v = 0; v < V; ++v) {
            work_side[v] = vside[v];
            dside[v] = vside[v];
        }
        const int32_t cross = (int32_t)((int64_t)H * (100 - dst_local_pct) / 100);
        for (int32_t i = 0; i < cross; ++i) {
            dside[hot0[H - 1 - i]] = 1;
            dside[hot1[H - 1 - i]] = 0;
            work_side[hot0[H - 1 - i]] = 1;
            work_side[hot1[H - 1 - i]] = 0;
        }
        for (int32_t v = 0; v < V; ++v) {
            rowptr[v] = v * degree;
            const int32_t *pool = dside[v] ? hot1 : hot0;
            for (int32_t j = 0; j < degree; ++j)
                col[(size_t)v * (size_t)degree + (size_t)j] =
                    pool[ora_splitmix64(seed, (uint64_t)v * (uint64_t)degree + (uint64_t)j) % (uint64_t)H];
        }
        rowptr[V] = V * degree;
        for (int32_t i = 0; i < nsrc; ++i) src[i] = (i & 1) ? hot1[(i / 2) % H] : hot0[(i / 2) % H];
    }
    free(hot0);
    free(hot1);
    free(vside);
    free(dside);
    return rc;
}

/* ------------------------------------------------------------------------------------ */
/* Dependent-probe hash (HASH.cu:29-83, 226-241)                                          */
/* ------------------------------------------------------------------------------------ */
int ora_dep_build(int32_t *table, uint64_t slots, const int32_t *keys, const int32_t *nexts, int32_t K,
                  uint64_t seed) {
    if ((uint64_t)K >= slots) return -1;
    const uint32_t mask = (uint32_t)(slots - 1);
    for (uint64_t s = 0; s < slots; ++s) {
        table[2 * s] = -1;
        table[2 * s + 1] = 0;
    }
    int32_t *perm = (int32_t *)malloc(sizeof(int32_t) * (size_t)K);
    if (!perm) return -2;
    for (int32_t i = 0; i < K; ++i) perm[i] = i;
    for (int64_t i = (int64_t)K - 1; i > 0; --i) {
        const int64_t j = (int64_t)(ora_splitmix64(seed, (uint64_t)i) % (uint64_t)(i + 1));
        const int32_t t = perm[i];
        perm[i] = perm[j];
        perm[j] = t;
    }
    for (int32_t k = 0; k < K; ++k) {
        const int32_t p = perm[k];
        uint32_t slot = ora_mix32((uint32_t)keys[p]) & mask;
        while (table[2 * (size_t)slot] != -1) slot = (slot + 1) & mask;
        table[2 * (size_t)slot] = keys[p];
        table[2 * (size_t)slot + 1] = nexts[p];
    }
    free(perm);
    return 0;
}

static int32_t dep_probe_one(const int32_t *table, uint32_t mask, int32_t key, int32_t *next_key) {
    uint32_t slot = ora_mix32((uint32_t)key) & mask;
    int32_t fkey = -1, fnext = key;
    for (uint64_t step = 0; step <= mask; ++step) {
        const int32_t ek = table[2 * (size_t)slot], en = table[2 * (size_t)slot + 1];
        if (ek == key) {
            fkey = ek;
            fnext = en;
            break;
        }
        if (ek == -1) break;
        slot = (slot + 1) & mask;
    }
    *next_key = fnext;
    return fkey == key ? (int32_t)slot : -1;
}

void ora_dep_probe(const int32_t *table, uint64_t slots, const int32_t *queries, int64_t n, int chain_len,
                   int32_t *out) {
    const uint32_t mask = (uint32_t)(slots - 1);
    for (int64_t i = 0; i < n; ++i) {
        int32_t key = queries[i];
        uint32_t acc = 0;
        for (int it = 0; it < chain_len; ++it) {
            int32_t nk;
            acc += (uint32_t)dep_probe_one(table, mask, key, &nk);
            key = nk;
        }
        out[i] = (int32_t)(acc ^ (uint32_t)key);
    }
}
