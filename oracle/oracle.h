/*
 * oracle.h -- CPU restatement of the reference's verification paths.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker (or the timed CPU
 * baseline). The product (libxdom, its runners and Python mirror) never links or calls it.
 *
 * Each function cites the reference code whose behaviour it restates.
 */
#ifndef XDOM_ORACLE_H
#define XDOM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

/* ---- generators (independent restatement of the build's seeded inputs) ---- */
uint64_t ora_splitmix64(uint64_t seed, uint64_t index);
uint32_t ora_mix32(uint32_t x); /* lowbias32 finaliser, GEMV.cu:56-63 */
uint16_t ora_f64_to_f16(double d);
double ora_f16_to_f64(uint16_t h);
void ora_gen_uniform_f32(float *out, size_t n, uint64_t seed);
void ora_gen_normal_f16(uint16_t *out, size_t n, double mean, double stddev, uint64_t seed);

/* ---- GEMV (GEMV.cu:383-402) ---- */
/* The reference's own check: fp32 running sum in k order. */
void ora_gemv_f32_seq(const float *A, const float *x, float *y, int64_t M, int64_t K, int nthreads);
/* fp64-accumulated y and the per-row magnitude sum |A_ik * x_k| (for relative bounds). */
void ora_gemv_f32_f64(const float *A, const float *x, double *y, double *yabs, int64_t M, int64_t K,
                      int nthreads);
void ora_gemv_f16_f64(const uint16_t *W, const uint16_t *x, double *y, double *yabs, int64_t M,
                      int64_t K, int nthreads);


/* ---- histogram (HIST.cu:279-299, generalised from 256 byte-bins to num_bins key bins) ---- */
/* Zipf(s) over num_bins ranks: t[k] = floor(2^64 * P(rank <= k)), t[num_bins-1] = 2^64-1. */
void ora_zipf_thresholds(uint64_t *t, uint32_t num_bins, double s);
/* key i = scramble(rank(splitmix64(seed, i))) with rank = least k, u < t[k]. */
void ora_gen_zipf_keys(uint32_t *keys, size_t n, const uint64_t *t, uint32_t num_bins, uint64_t seed,
                       int scramble);
uint32_t ora_zipf_scramble(uint32_t rank, uint32_t num_bins);
uint32_t ora_zipf_key_at(const uint64_t *t, uint32_t num_bins, uint64_t seed, int scramble, uint64_t index);
/* counts[k] = #{i : keys[i] == k}; keys >= num_bins are not counted. Returns the number counted. */
uint64_t ora_histogram(const uint32_t *keys, size_t n, uint32_t *counts, uint32_t num_bins, int nthreads);

/* The reference's own histogram (HIST.cu:279-288, 331-340): words[i] = mix32(i ^ seed), every
 * byte of every word counted into 256 bins (nthreads private histograms, summed). */
void ora_gen_mix32_words(uint32_t *out, size_t n, uint32_t seed);
void ora_hist256_bytes(const uint32_t *words, size_t n, uint32_t *counts, int nthreads);
/* GEMV init_data (GEMV.cu:118-139): (h & 0xff) / 255 - 0.5 (modulus 0) or h % modulus - offset. */
void ora_gen_mix32_f32(float *out, size_t n, uint32_t seed, uint32_t modulus, int32_t offset);

/* ---- hash table (HASH.cu:46-64 probe, HASH.cu:226-241 serial CPU insert; u64 keys+values) ---- */
uint64_t ora_mix64(uint64_t z); /* splitmix64 output function */
void ora_hash_kv(uint64_t *keys, uint64_t *vals, uint64_t n, uint64_t seed);
void ora_hash_queries(uint64_t *q, uint64_t n, uint64_t n_keys, uint64_t seed, uint64_t qseed);
/* Serial insert in input order into tkeys/tvals (slots entries, tkeys preset by the function
 * to EMPTY). Returns the number of pairs that found no slot within min(slots, 65536). */
uint64_t ora_hash_build(uint64_t *tkeys, uint64_t *tvals, uint64_t slots, const uint64_t *keys,
                        const uint64_t *vals, uint64_t n);
void ora_hash_lookup(const uint64_t *tkeys, const uint64_t *tvals, uint64_t slots, const uint64_t *q,
                     uint64_t n, uint64_t *vals_out, uint8_t *found_out, int nthreads);

/* ---- BFS (bfs.cu:215-252 level rule: depth + 1 at the first visit, 0xFFFFFFFF unvisited) ---- */
void ora_rmat_edge(int scale, double a, double b, double c, uint64_t seed, uint64_t e, int32_t *u, int32_t *v);
/* Undirected CSR (both directions, no self-loops, no duplicates, sorted lists); returns nnz.
 * col must hold 2 * edge_factor * 2^scale entries. */
int64_t ora_rmat_csr(int scale, int edge_factor, double a, double b, double c, uint64_t seed, int32_t *rowptr,
                     int32_t *col);
/* Serial FIFO-queue BFS; returns the number of reached vertices. */
int64_t ora_bfs(const int32_t *rowptr, const int32_t *col, int32_t V, int32_t src, uint32_t *level);
/* The reference's workload: multi-source BFS limited to max_depth levels over a directed graph
 * (bfs.cu:151-252, 449-491), and its hot-pool graph (bfs.cu:354-409). */
int64_t ora_bfs_multi(const int32_t *rowptr, const int32_t *col, int32_t V, const int32_t *src, int32_t nsrc,
                      int32_t max_depth, uint32_t *level);
int ora_bfs_ref_graph(int32_t V, int32_t degree, int32_t nsrc, int32_t dst_local_pct, int32_t H, uint64_t seed,
                      uint64_t col_addr, const uint8_t *col_home, uint64_t level_addr, const uint8_t *level_home,
                      uint64_t mask, int32_t *rowptr, int32_t *col, uint8_t *work_side, int32_t *src);

/* The reference's dependent-probe workload (applications/hash/src/hash_probe_dep.cu).
 * ora_dep_build: table[2*slots] {key, next}, EMPTY -1, serial insertion (HASH.cu:232-241) in
 * the order of a Fisher-Yates shuffle (i = K-1 .. 1, j = splitmix64(seed, i) mod (i + 1)).
 * ora_dep_probe: probe_dep_base (HASH.cu:66-83) with probe_chain_one (:46-64), int wraps. */
int ora_dep_build(int32_t *table, uint64_t slots, const int32_t *keys, const int32_t *nexts, int32_t K,
                  uint64_t seed);
void ora_dep_probe(const int32_t *table, uint64_t slots, const int32_t *queries, int64_t n, int chain_len,
                   int32_t *out);

#endif
