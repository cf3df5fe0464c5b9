/*
 * xdom.h -- C ABI of libxdom, the MI355X (gfx950) XCD-domain kernel library.
 *
 * The reference (LyleLuo/L2Domain) has no library interface: its hot kernels are
 * file-local `__global__` functions inside one executable per application, driven by
 * positional argv and parsed from stdout. This header is the drop-in boundary that
 * replaces those kernels; each entry point names the reference code it stands in for.
 *
 * Conventions (all entry points):
 *   - Plain C types only. Device buffers are caller-owned device pointers; `stream` is a
 *     hipStream_t passed as void* (NULL = the null stream).
 *   - Return 0 (XD_OK) on success, a negative XD_ERR_* code on failure. Nothing aborts.
 *     xd_last_error() gives a human-readable message for the calling thread.
 *   - `mode` selects the work placement:
 *       XD_MODE_OBLIVIOUS  default dispatch order, no XCD awareness (the reference's
 *                          "baseline", e.g. gemv_baseline_kernel GEMV.cu:199-231);
 *       XD_MODE_AWARE      every XCD owns one contiguous slice of the data (the reference's
 *                          "aware", e.g. gemv_partitioned_kernel GEMV.cu:163-197);
 *       XD_MODE_ROTATED    negative control, the reference's "swapped" (GEMV.cu:176): data
 *                          is handled away from its domain -- by the other I/O die for the
 *                          memory-home-routed kernels (hash), by XCD (s+r) mod 8 for the
 *                          slice-routed ones, r advancing by one on every pass.
 *   - Entry points that need scratch memory take a caller-owned workspace whose size is
 *     given by the matching *_workspace_size() query (the reference's nullptr -> bytes
 *     size-query idiom, utility/latopt.cuh:532-540). A workspace must be zeroed once
 *     after allocation (hipMemset to 0); the kernels leave it zeroed again on exit.
 *   - Work is stream-ordered; functions return after enqueueing unless stated otherwise.
 */
#ifndef XDOM_H
#define XDOM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define XD_OK 0
#define XD_ERR_INVALID_ARG (-1)
#define XD_ERR_HIP (-2)
#define XD_ERR_WORKSPACE (-3)
#define XD_ERR_UNSUPPORTED (-4)
#define XD_ERR_TABLE_FULL (-5)
#define XD_ERR_INCOMPLETE (-6)

#define XD_MODE_OBLIVIOUS 0
#define XD_MODE_AWARE 1
#define XD_MODE_ROTATED 2

#define XD_NUM_XCD 8

/* ------------------------------------------------------------------------------------ */
/* Library, topology and domain runtime                                                  */
/* ------------------------------------------------------------------------------------ */

typedef struct {
    int device;
    int num_cu;               /* compute units visible to the process            */
    int num_xcd;              /* XCDs (L2 domains); 8 on MI355X in SPX mode       */
    int cu_per_xcd;
    int wave_size;            /* 64 on CDNA                                      */
    int clock_khz;            /* shader clock                                     */
    long long l2_bytes;       /* L2 size reported by the runtime (per XCD on CDNA) */
    long long lds_bytes_per_wg;
    long long hbm_bytes;
    char arch[32];            /* e.g. "gfx950:sramecc+:xnack-"                   */
    char name[96];
} xd_topology_t;

/* Library version string. */
const char *xd_version(void);

/* Message describing the last error raised on the calling thread ("" if none). */
const char *xd_last_error(void);

/* Per-kernel timing of the library's own launches, for benchmarks: when enabled, every
 * kernel dispatch stamps a start/stop HIP event pair itself (hipExtLaunchKernel), so a
 * kernel's time is its own execution, without the gaps between dispatches; kernels are
 * named after their __global__ functions. xd_timing_enable resets
 * the accumulators; xd_timing_query(i, ...) reports kernel number i (in first-launch order)
 * with its summed duration and launch count, waiting for outstanding launches; it returns
 * XD_ERR_INVALID_ARG past the last kernel. No counterpart in the reference (which times
 * whole kernels with cudaEvent pairs in each main(), e.g. GEMV.cu:301-316). */
int xd_timing_enable(int on);
int xd_timing_query(int index, char *name, int name_len, double *total_ms, long long *launches);

/* Static description of the device. Replaces the latency-probed SM->side map
 * latopt::get_map_smid2side (utility/latopt.cuh:487-562): on CDNA the L2 domain of a
 * workgroup is read from the hardware (HW_REG_XCC_ID), so nothing has to be probed. */
int xd_topology_query(int device, xd_topology_t *out);

/* DomainScan: launch `num_wg` workgroups and record, for each, the hardware placement
 * word ((xcc_id << 24) | (se_id << 16) | (sh_id << 12) | (cu_id << 8) | simd_id) into
 * out_placement[wg] (device buffer of num_wg uint32). Evidence for the workgroup->XCD
 * dispatch order the XCD-aware kernels assume. Stands in for the reference's SM->side
 * calibration (utility/get_smid2side.cu:73-112, utility/latopt.cuh:487-530). */
int xd_domain_scan(int num_wg, uint32_t *out_placement, void *stream);

/* The XCD that workgroup 0 of the last dispatch of this library's kernels on `stream` (on the
 * current device) ran on, or -1 before the first. A dispatch's workgroup i runs on XCD
 * (i + offset) mod 8, the offset fixed per hardware queue: 0 on the queues a process uses
 * first, other values on queues mapped later (measured with xd_domain_scan on nine
 * streams). Every XCD-aware kernel places its work for the offset its stream last reported
 * and reports its own, so placement is right from the second call on a stream; results
 * never depend on it. No counterpart in the reference, whose kernels read the SM id
 * (__smid) themselves (utility/latopt.cuh:487-530). */
int xd_xcd_offset(void *stream);

/* Memory home of an address: MI355X (SPX/NPS1) spreads memory over two I/O dies; XCDs 0-3
 * sit next to die 0 and XCDs 4-7 next to die 1. The die homing the 8 KiB chunk at byte
 * address a is popcount(a & mask) & 1, with mask = 0x10202000 (bits 13, 21, 28) by default
 * (measured: near lines ~850 cycles from HBM / ~520 from the Infinity Cache, far lines
 * ~1070 / ~740). Same form as the reference's side prediction
 * predict_map_memory_attr_far (utility/latopt.cuh:255-263), with a fixed instead of a
 * per-page attribute. The home-routed kernels (hash, GEMV row segments) use this mask when
 * no page map is passed. Any non-zero mask of bits at or above 13 is accepted; one without
 * bit 13 can put both 8 KiB chunks of a 16 KiB pair on one die, and the hash bulk build then
 * takes its contiguous ranges instead of die halves (the other routes read every chunk once
 * under any mask, near or not). */
uint64_t xd_home_mask(void);
int xd_set_home_mask(uint64_t mask);

/* MaskProbe / page attributes. Address bits above the 2 MiB page come from the physical
 * placement of the page, so the die of a page is measured: for every 2 MiB page overlapping
 * [buf, buf + bytes), XCD 0 (die 0) and then XCD 4 (die 1) time a fetch-add of 0 (the data
 * is left unchanged) on words at page offsets 0, 16, 32, 48 KiB (all with bit 13 = 0);
 * atomics execute beyond the L2 on gfx950, so the faster die is the home: attr[p] = 1 if
 * die 1 was faster, else 0. The buffer must not be written concurrently. The home of address
 * a is then bit13(a) ^ attr[a / 2 MiB - buf / 2 MiB]. Replaces the reference's per-page
 * attribute probe get_map_memory_attr (utility/latopt.cuh:683-814). attr and workspace
 * are device buffers of xd_home_map_pages() bytes and xd_home_map_workspace_size() bytes. */
size_t xd_home_map_pages(const void *buf, size_t bytes);
size_t xd_home_map_workspace_size(const void *buf, size_t bytes);
int xd_home_map(const void *buf, size_t bytes, uint8_t *attr, void *workspace, size_t workspace_bytes,
                void *stream);

/* XDom-PChase. Builds a pointer chain of numel (2..8192) 8-byte elements at a stride of
 * stride_bytes in `chain` (device, >= numel * stride_bytes), optionally evicts the caches by
 * streaming flush_buf (NULL: no flush), then a workgroup on XCD leader_xcd chases the chain
 * twice and, after that launch ends, a workgroup on XCD follower_xcd chases it twice. One
 * lane times every dependent load with s_memtime. out (device, 4 * numel + 4 uint32):
 * [0, n) leader first, [n, 2n) leader second, [2n, 3n) follower first, [3n, 4n) follower
 * second (cycles), then the leader's and follower's XCC ids and two claim words that read 1
 * when each role found its XCD. Same protocol as k_peer_pchase / run_figure_2
 * (utility/latopt.cuh:354-406, architecture/src/architecture_probe.cu:572-596) with XCDs in
 * place of SMs and a kernel boundary in place of the leader -> follower flag. */
int xd_xdom_pchase(int leader_xcd, int follower_xcd, void *chain, size_t chain_bytes, int numel, int stride_bytes,
                   const void *flush_buf, size_t flush_bytes, uint32_t *out, void *stream);

/* MaskProbe. For the base address buf and buf + 2^b, b = first_bit..last_bit (buf device,
 * >= 2^last_bit + 4 bytes, zero or any data: it is left unchanged), a workgroup on XCD 0
 * (I/O die 0) and then one on XCD 4 (die 1) record the minimum over `reps` returning
 * memory-side fetch-adds of 0. out (device, 2 * nb + 4 uint32 with nb = last_bit -
 * first_bit + 2): [0, nb) die-0 cycles (entry 0 = base, entry k = bit first_bit + k - 1),
 * [nb, 2nb) die-1 cycles, then the two XCC ids and two claim words. A bit is active where
 * the die-0 / die-1 latency relation differs from the base address's (derive_active_bits,
 * architecture/src/architecture_probe.cu:495-523, run_mask_probe :644-670); only bits
 * below 21 are page-stable (2 MiB pages). */
int xd_mask_probe(void *buf, size_t bytes, int first_bit, int last_bit, int reps, uint32_t *out, void *stream);

/* DomainScan latency curves (run_figure_3, architecture/src/architecture_probe.cu:598-631,
 * on measure_offsets :417-458): after a cache flush (flush_buf of xd_cache_flush_bytes(), or
 * NULL for none), the first workgroup on XCD `leader_xcd` loads buf + 2^b for b in
 * [first_bit, last_bit]; then the first workgroup running on the compute unit `follower_cu`
 * times one load of each address, in that order. follower_cu is a placement key
 * (xcc << 16) | (se << 8) | (sh << 4) | cu: an xd_domain_scan word shifted right by 8. The
 * leader hands over at the kernel boundary (L2 and Infinity Cache contents survive it). out
 * (device, uint32): [last_bit - first_bit + 1] follower cycles, then [leader found, follower
 * found, leader XCC, 0]: a 0 in either flag means no workgroup ran there and the curve is
 * unwritten. buf: device, 8-byte aligned, at least 2^last_bit + 8 bytes. */
int xd_domain_scan_latency(void *buf, size_t bytes, int first_bit, int last_bit, int leader_xcd, uint32_t follower_cu,
                           const void *flush_buf, size_t flush_bytes, uint32_t *out, void *stream);

/* Channel probe, the MaskProbe search for the address bits that select an L2 channel of an
 * XCD (measure_offsets / run_mask_probe, architecture/src/architecture_probe.cu:417-458,
 * 644-686; k_get_mask, utility/get_mask.cu:87-150, which find the bits that pick an H100 L2
 * partition). A query times a set of 64 lines: lane i of 128 one-wave workgroups on XCD
 * `xcd` reads base + (XOR of vecs[k] over the set bits k of i), `iters` times, with loads
 * that skip the vector L1 and hit the L2. A channel serves its lines one after another, so
 * the time grows with the largest number of lines sharing a channel. base = buf rounded up to
 * 2 MiB (buf device; bytes must still cover the span after the rounding). Times are HIP-event
 * minima of three launches on `stream`; the calls wait for them.
 *
 * xd_channel_time: one query. vecs (host, 6 entries): multiples of 128 below 2^40.
 *
 * xd_channel_probe: recovers the channel-select functions as XOR masks of address bits in
 * [bit0, bit1] (7 <= bit0, bit0 + 6 <= bit1 < 34). out_window_us[bit1 - bit0 - 4]: the windows
 * of six consecutive bits b..b+5, b = bit0.. ; out_fast_us: the fastest time seen (every
 * channel in use). Then up to max_sets five-bit sets F in a fixed pseudo-random order: a set
 * whose image has rank one below the maximum gives, per added bit f, T_fast when f is in the
 * mask of the one channel function that is constant on F, 2 T_fast otherwise. Each new mask
 * (GF(2)-independent of those found) goes to out_masks[k] (up to 4) with its curve
 * out_curves[k * (bit1 - bit0 + 1) + (f - bit0)] (microseconds; 0 for the bits of F);
 * *out_nmasks = how many. */
int xd_channel_time(void *buf, size_t bytes, int xcd, const uint64_t *vecs, int iters, float *out_us, void *stream);
int xd_channel_probe(void *buf, size_t bytes, int xcd, int bit0, int bit1, int iters, int max_sets,
                     float *out_window_us, float *out_fast_us, uint64_t *out_masks, float *out_curves, int *out_nmasks,
                     void *stream);

/* Memory-side channel probe, the MaskProbe search beyond the L2 (same reference functions as
 * xd_channel_probe): every workgroup of a 2048-wave grid (all XCDs) adds 1 to the same set of
 * 64 lines, base + (XOR of vecs[k] over the set bits k of the lane), wave w at dword
 * (w mod 16) * 8 of each line, `iters` times; a line's returning atomic is served by one
 * memory-side unit, so the time grows with the largest number of the set's lines sharing one
 * (it doubles per dimension the set's image loses). The adds change the buffer. base = buf
 * rounded up to 2 MiB; buf device, bytes must cover the span after the rounding.
 *
 * xd_memchannel_time: one query (vecs: 6 host entries, multiples of 128 below 2^40).
 *
 * xd_memchannel_probe: over address bits [bit0, bit1] (7 <= bit0, bit0 + 6 <= bit1 < 34, at
 * most 32 bits), every single bit and every pair of bits x is tried against `nsets` seeded
 * five-vector sets F: out_ratio[a * nb + b] (a <= b, a == b the single bit, nb = bit1 - bit0
 * + 1; host, nb * nb floats) = min over the sets of time(F + x) / the fastest time of F's
 * curve. A ratio near 1 means x spread the set over more units for some F; near 2 or more,
 * x never changes the unit. *out_inactive: the bits that never do; out_masks[0 .. *out_nmasks)
 * (host, up to 32): the remaining bits grouped into classes of equal image (pairs that never
 * change the unit), one XOR mask per class -- the unit-select functions when every bit enters
 * exactly one of them, which the GPU test checks by predicting random sets. */
int xd_memchannel_time(void *buf, size_t bytes, const uint64_t *vecs, int iters, float *out_us, void *stream);
int xd_memchannel_probe(void *buf, size_t bytes, int bit0, int bit1, int iters, int nsets, float *out_ratio,
                        uint64_t *out_inactive, uint64_t *out_masks, int *out_nmasks, void *stream);

/* Bytes of read traffic xd_cache_flush needs to evict 8 x 4 MB L2 and the 256 MB
 * Infinity Cache (>= 4x their sum). */
size_t xd_cache_flush_bytes(void);

/* Stream-read `bytes` of `buf` (device, >= xd_cache_flush_bytes()) so that previously
 * touched data is no longer cache resident. Replaces GlobalL2Cache::reset
 * (utility/latopt.cuh:103-134) and flush_l2_k (histogram256_sideaware.cu:39-49), which
 * size the flush from cudaDeviceProp::l2CacheSize. */
int xd_cache_flush(const void *buf, size_t bytes, void *stream);

/* Read `bytes` of `buf` (device) once, 16 bytes per load, and discard the words: the
 * roofline probe of cache-resident workloads (the warm GEMV configurations). Oblivious:
 * contiguous; XD_MODE_AWARE: each I/O die reads only the 8 KiB chunks it homes (home_attr =
 * xd_home_map() of buf, or NULL for the address-mask prediction; buf and bytes in whole
 * 16 KiB pairs); XD_MODE_ROTATED: only the far chunks. Launch shape: `workgroups` (a
 * multiple of 8; 0 = 2048) of 256 threads, each thread keeping 2 x `depth` (1, 2, 4 or 8;
 * 0 = 4) loads in flight. No counterpart in the reference, whose warm runs (touch_k,
 * histogram256_sideaware.cu:27-37) have no bandwidth ceiling. */
int xd_read_stream(const void *buf, size_t bytes, int mode, const uint8_t *home_attr, int workgroups, int depth,
                   void *stream);

/* ------------------------------------------------------------------------------------ */
/* GEMV  y[M] = A[M,K] . x[K], row-major A, fp32 accumulation                            */
/* ------------------------------------------------------------------------------------ */

/* Workspace bytes the GEMV entry points use for the split-row home routing of an M x K
 * matrix of elem_bytes (4: fp32, 2: fp16) elements: M * (S + 1) * 4 when a row is S >= 2
 * whole 8 KiB chunks (rows <= 64 KiB), else 0 (no workspace used). No counterpart in the
 * reference (its rows never span two sides' memory, GEMV.cu:264-273). */
size_t xd_gemv_workspace_size(int M, int K, int elem_bytes);

/* fp32 GEMV. Replaces gemv_partitioned_kernel / gemv_baseline_kernel
 * (applications/gemv/src/gemv_k1024_persistent_subwarp.cu:163-231), generalised from the
 * compile-time K=1024 to any K with K % 4 == 0 and 16-byte aligned A and x.
 * Writes every y[i] (no accumulation into y). Placement:
 *   XD_MODE_OBLIVIOUS  row chunks go to workgroups in order (consecutive chunks land on
 *                      different XCDs);
 *   XD_MODE_AWARE      with A 8 KiB aligned, work follows memory homes (home_attr =
 *                      xd_home_map() of A; NULL = the address-mask prediction):
 *                      rows that divide 8 KiB go whole to the I/O die homing them; rows of
 *                      S >= 2 whole 8 KiB chunks are split into their chunks, each reduced
 *                      on its home die and combined in chunk order (needs a workspace of
 *                      xd_gemv_workspace_size() bytes, 8-byte aligned, zero-filled once when
 *                      allocated; each call leaves it zeroed; calls sharing one workspace
 *                      must not overlap).
 *                      Otherwise (rows that straddle 8 KiB chunks, no workspace, A not
 *                      8 KiB aligned) no die placement applies and the rows keep the
 *                      oblivious order, which measured faster than one contiguous eighth
 *                      of the rows per XCD;
 *   XD_MODE_ROTATED    the home routes with the far die; otherwise each XCD takes a
 *                      rotated contiguous eighth of the rows (the "swapped" control).
 * The split-row route gives bit-identical y to XD_MODE_OBLIVIOUS for S = 2 and 4. */
int xd_gemv_f32(const float *A, const float *x, float *y, int M, int K, int mode, const uint8_t *home_attr,
                void *workspace, size_t workspace_bytes, void *stream);

/* fp16 weights and vector (IEEE binary16 bit patterns), fp32 accumulation, fp32 y.
 * Same structure as xd_gemv_f32; K % 8 == 0, 16-byte aligned W and x. */
int xd_gemv_f16f32(const uint16_t *W, const uint16_t *x, float *y, int M, int K, int mode,
                   const uint8_t *home_attr, void *workspace, size_t workspace_bytes, void *stream);

/* ------------------------------------------------------------------------------------ */
/* Histogram  counts[k] = #{i : keys[i] == k}, k < num_bins                               */
/* ------------------------------------------------------------------------------------ */

/* Workspace bytes xd_hist_u32 needs for n keys and num_bins counters (0 if num_bins is out
 * of range). About 2 bytes per key, 1 KiB per 24576-key tile (hot-key counters) and 128 KB
 * per counting workgroup. The workspace must be
 * zero-filled once when allocated; every call leaves its counters zeroed again, and a
 * workspace sized for n keys serves any smaller n. Calls sharing one workspace must not
 * overlap. */
size_t xd_hist_workspace_size(size_t n, uint32_t num_bins);

/* Histogram of uint32 keys into num_bins (1..2^24) uint32 counters; keys >= num_bins are
 * not counted. Every counts[k] is written (no accumulation into counts). n < 2^32. Calls of
 * at least 2^20 keys into at most 2^20 bins first sample the keys for up to 256 frequent
 * ones, which are counted in LDS during the partition (one more launch; the counts do not
 * depend on which keys it picks).
 * Replaces histogram256_chunked_kernel / histogram256_persistent_kernel /
 * merge_histogram256_kernel (applications/histogram/src/histogram256_sideaware.cu:51-157),
 * generalised from 256 byte-bins (add_word, :20-25) to one bin per key. XD_MODE_AWARE
 * has each I/O die read only the 8 KiB key chunks it homes (as the reference's side-aware
 * chunks do; home_attr = xd_home_map() of the keys, device, optional: NULL = the
 * address-mask prediction) and range-partitions the bins over the XCDs for counting: XCD
 * x counts only its bin range (the final merge runs over the whole grid in every mode).
 * XD_MODE_ROTATED reads the far chunks and counts each range on another XCD. An error
 * returned after the first kernel was enqueued (a HIP launch failure) leaves the workspace
 * dirty: zero-fill it again before the next call. */
int xd_hist_u32(const uint32_t *keys, size_t n, uint32_t *counts, uint32_t num_bins, int mode,
                const uint8_t *home_attr, void *workspace, size_t workspace_bytes, void *stream);

/* Workspace bytes of xd_hist256_u32bytes (independent of n: 8448 bytes of accumulators and
 * tickets). Zero-filled once when allocated; every call leaves it zeroed again. Calls
 * sharing one workspace must not overlap. */
size_t xd_hist256_workspace_size(void);

/* The reference's own histogram: 256 byte-bins, every byte of every word counted,
 * counts[v] = #{(i, k) : (words[i] >> 8k) & 0xff == v}; all 256 counts are written.
 * words 16-byte aligned, n < 2^30. Replaces add_word / histogram256_chunked_kernel /
 * histogram256_persistent_kernel / merge_histogram256_kernel
 * (applications/histogram/src/histogram256_sideaware.cu:20-25, 51-157) with the near/far
 * chunk lists of :227-277. Modes: XD_MODE_OBLIVIOUS reads every 8 KiB chunk from any XCD;
 * XD_MODE_AWARE has each I/O die read only the chunks it homes (home_attr: xd_home_map of
 * words, or NULL for the address-mask prediction); XD_MODE_ROTATED only the far chunks. */
int xd_hist256_u32bytes(const uint32_t *words, size_t n, uint32_t *counts, int mode, const uint8_t *home_attr,
                        void *workspace, size_t workspace_bytes, void *stream);

/* xd_hist256_u32bytes without a caller workspace and without any allocation: for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference. The accumulators and
 * tickets live in a fixed library array of 8448 bytes per GPU (held until the process ends),
 * set up and zero-filled on the first call on each device and left zeroed by every call;
 * the limits are those of xd_hist256_u32bytes (n < 2^30 words), larger inputs are refused
 * with XD_ERR_INVALID_ARG. Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (other streams, other host threads) race and must be serialised by the
 * caller. Never timed by xd_timing_enable (it creates no events). */
int xd_hist256_u32bytes_noalloc(const uint32_t *words, size_t n, uint32_t *counts, int mode,
                                const uint8_t *home_attr, void *stream);

/* ------------------------------------------------------------------------------------ */
/* Hash table: open addressing, linear probing, uint64 keys and values                   */
/* ------------------------------------------------------------------------------------ */
/* Layout: `slots` (a power of two) 16-byte slots {uint64 key; uint64 value}; a key equal to
 * XD_HASH_EMPTY marks a free slot. The home slot of key k is splitmix64_mix(k) & (slots-1)
 * (the splitmix64 output function, a bijection) and probing walks forward with wrap-around,
 * at most min(slots, 65536) slots. Same probe structure as probe_chain_one
 * (applications/hash/src/hash_probe_dep.cu:46-64: mix32(key) & mask, stop at the key or at
 * EMPTY), widened to 64-bit keys with values, and with GPU insertion in place of the
 * reference's serial CPU build (:226-241).
 * Modes: XD_MODE_OBLIVIOUS walks the keys in launch order (probe_dep_base, :66-83);
 * XD_MODE_AWARE lets the XCDs of each I/O die take only the keys whose home slot is homed
 * on that die (xd_home_mask), like probe_dep_sa (:85-116) with per-side routing (:244-270)
 * but filtered on the device; XD_MODE_ROTATED hands each die the other die's keys (the
 * reference's swapped launch, :317-323). */
#define XD_HASH_EMPTY 0xFFFFFFFFFFFFFFFFull

size_t xd_hash_table_bytes(uint64_t slots);

/* Marks every slot free. */
int xd_hash_init(void *table, uint64_t slots, void *stream);

/* Inserts n (key, value) pairs; an existing key gets the new value (duplicates inside one
 * call keep one of their values). Keys equal to XD_HASH_EMPTY are skipped. Pairs that find
 * no free slot within the probe limit are counted into *failed (device counter, optional).
 * home_attr: xd_home_map() of the table (device, optional; NULL = xd_home_mask()), used by
 * the aware and rotated modes to tell which die homes a slot. Results never depend on it. */
int xd_hash_insert_u64(void *table, uint64_t slots, const uint64_t *keys, const uint64_t *vals, uint64_t n,
                       int mode, const uint8_t *home_attr, unsigned long long *failed, void *stream);

/* Bulk build: the table's previous contents are replaced by the n pairs (the insert's
 * semantics on a freshly cleared table: EMPTY keys skipped, a repeated key keeps one of its
 * values, pairs that find no slot counted into *failed). No counterpart routine in the
 * reference, which builds its table serially on the CPU
 * (applications/hash/src/hash_probe_dep.cu:226-241); this is that build on the GPU. Tables of
 * 2^15 .. 2^30 slots are built range by range in LDS (4096 slots per range, two split passes,
 * plain stores, a compare-and-swap fix-up for the few pairs that run past a range's end);
 * XD_MODE_AWARE makes a range the 8 KiB chunks homed on one I/O die and builds it on that
 * die, XD_MODE_ROTATED on the other die. Other sizes, n = 0 and calls of fewer than
 * slots / 64 pairs are cleared and inserted (xd_hash_init + xd_hash_insert_u64). The
 * workspace (xd_hash_build_workspace_size, 0 for those shapes) needs no initial contents; it
 * is about 3.1 n x 16 bytes at load factors near 0.5 and at most about 7 n x 16 bytes (each
 * range's regions have a floor of ~2 x 72 pairs plus 32 spill slots). */
size_t xd_hash_build_workspace_size(uint64_t n, uint64_t slots);
int xd_hash_build_u64(void *table, uint64_t slots, const uint64_t *keys, const uint64_t *vals, uint64_t n,
                      int mode, const uint8_t *home_attr, void *workspace, size_t workspace_bytes,
                      unsigned long long *failed, void *stream);

/* found_out[i] = 1 and vals_out[i] = value if queries[i] is present, else 0 and 0. */
int xd_hash_lookup_u64(const void *table, uint64_t slots, const uint64_t *queries, uint64_t n,
                       uint64_t *vals_out, uint8_t *found_out, int mode, const uint8_t *home_attr,
                       void *stream);

/* Device generators: keys[i] = xd_rand64(seed, i) (distinct), vals[i] =
 * xd_rand64(seed ^ 0x5BD1E9955BD1E995, i) (vals may be NULL); query j is the key of index
 * xd_rand64(qseed, j) mod n_keys for even j (a hit) and of index n_keys + j/2 for odd j
 * (a miss: outside the inserted range). */
int xd_gen_hash_kv(uint64_t *keys, uint64_t *vals, uint64_t n, uint64_t seed, void *stream);
int xd_gen_hash_queries(uint64_t *queries, uint64_t n, uint64_t n_keys, uint64_t seed, uint64_t qseed,
                        void *stream);

/* The reference's own hash workload (applications/hash/src/hash_probe_dep.cu), as an input
 * mode: a table of `slots` 8-byte entries {int32 key; int32 next} (EMPTY key = -1), home slot
 * mix32(key) & (slots - 1) (lowbias32), linear probing.
 * xd_dep_make_keys (host): K keys with successors -- two hot pools of H odd keys whose home
 *   slots lie on I/O die 0 and die 1 of the table at device address table_addr (home_attr_host
 *   = a host copy of xd_home_map() of the table, NULL = address-mask prediction), each chained
 *   into a cycle, then cold keys that are their own successor (HASH.cu:194-224).
 * xd_dep_build (host): table[2 * slots] filled by serial insertion in the order of a
 *   Fisher-Yates shuffle driven by xd_rand64(seed, i) (HASH.cu:226-241).
 * xd_dep_queries (host): the first hot_pct percent of the Q queries alternate the hot pools
 *   (even: die-0 pool), the rest are uniform over all keys (HASH.cu:244-270).
 * xd_dep_probe (device): out[i] = (sum over chain_len dependent probes of the found slot, or
 *   -1 for a missing key, wrapping) ^ the final key (probe_chain_one / probe_dep_base,
 *   HASH.cu:46-83). XD_MODE_AWARE routes every query to the die that homes its first slot
 *   (probe_dep_sa with per-side query lists, :85-116, with the routing done on the device);
 *   XD_MODE_ROTATED to the other die. home_attr: xd_home_map() of the table (device). */
int xd_dep_make_keys(uint64_t table_addr, uint64_t slots, const uint8_t *home_attr_host, int32_t K, int32_t H,
                     int32_t *keys, int32_t *nexts);
int xd_dep_build(int32_t *table, uint64_t slots, const int32_t *keys, const int32_t *nexts, int32_t K,
                 uint64_t seed);
int xd_dep_queries(int32_t *queries, int32_t Q, const int32_t *keys, int32_t K, int32_t H, int32_t hot_pct,
                   uint64_t seed);
int xd_dep_probe(const void *table, uint64_t slots, const int32_t *queries, uint64_t n, int chain_len,
                 int32_t *out, int mode, const uint8_t *home_attr, void *stream);

/* The reference's routed form of the dependent probe, with the routing as its own step:
 * xd_dep_route (device) partitions the queries, in order, into two lists of {key, query id}
 * by the I/O die homing each query's first slot (the near/far lists the reference builds on
 * the host, HASH.cu:244-270, outside its timed region); route is a device buffer of
 * xd_dep_route_bytes(n) bytes, 16-byte aligned. xd_dep_probe_routed (device) runs
 * probe_dep_sa (HASH.cu:85-116): die d probes list d (XD_MODE_AWARE) or list 1 - d
 * (XD_MODE_ROTATED; XD_MODE_OBLIVIOUS: every workgroup takes both lists) and writes
 * out[query id] exactly as xd_dep_probe does. n < 2^31. The route stays valid for the same
 * table, queries and home map. */
size_t xd_dep_route_bytes(uint64_t n);
int xd_dep_route(const void *table, uint64_t slots, const int32_t *queries, uint64_t n, const uint8_t *home_attr,
                 void *route, size_t route_bytes, void *stream);
int xd_dep_probe_routed(const void *table, uint64_t slots, const void *route, uint64_t n, int chain_len,
                        int32_t *out, int mode, void *stream);

/* ------------------------------------------------------------------------------------ */
/* BFS over an undirected CSR graph                                                       */
/* ------------------------------------------------------------------------------------ */
typedef struct {
    int32_t levels;           /* distinct BFS levels (max level + 1)                    */
    int32_t topdown_steps;
    int32_t bottomup_steps;
    int64_t reached_vertices;
    int64_t reached_edges;    /* sum of the degrees of the reached vertices (TEPS = /2) */
} xd_bfs_stats_t;

size_t xd_bfs_workspace_size(int32_t num_vertices, int64_t nnz);

/* Route of a graph for the XCD-aware and rotated BFS modes: the 64-vertex blocks sorted by
 * the I/O die that homes the start of their adjacency in col (home_attr = xd_home_map() of
 * col, device; NULL = the address-mask prediction). It depends only on the graph and where
 * col lives, so it is built once per graph, like the reference's per-vertex work_side map
 * (applications/bfs/src/bfs.cu:354-409), and reused by every search; rebuild it if col
 * moves. route: device buffer of xd_bfs_route_bytes(V) bytes, 16-byte aligned. */
size_t xd_bfs_route_bytes(int32_t num_vertices);
int xd_bfs_route(const int32_t *rowptr, const int32_t *col, int32_t num_vertices, int64_t nnz,
                 const uint8_t *home_attr, void *route, size_t route_bytes, void *stream);

/* level[v] = BFS distance from src, XD_BFS_UNVISITED (0xFFFFFFFF) if unreachable, for the
 * undirected graph rowptr[V+1] / col[nnz] (int32, device; every edge stored both ways).
 * Direction-optimizing (top-down and bottom-up steps over frontier bitmaps, Beamer's switch with
 * alpha = 14 and beta = 24, decided on the device; the host reads the control block after six
 * levels and then after every four). Replaces luo_baseline_level_kernel / luo_side_level_kernel and the host
 * level loops (applications/bfs/src/bfs.cu:215-308, 449-491), which run a fixed number of
 * top-down levels from many sources; the level values follow the same rule (depth + 1 at the
 * first claim, :240, 0xFFFFFFFF unvisited, :30). Modes act on the bottom-up steps:
 * XD_MODE_OBLIVIOUS walks 64-vertex blocks in order; XD_MODE_AWARE gives each I/O die the
 * blocks of its route list (route from xd_bfs_route(); NULL = built in this call with the
 * address-mask prediction); XD_MODE_ROTATED gives each die the other die's blocks. */
#define XD_BFS_UNVISITED 0xFFFFFFFFu
int xd_bfs_csr(const int32_t *rowptr, const int32_t *col, int32_t num_vertices, int64_t nnz, int32_t src,
               uint32_t *level, int mode, const void *route, void *workspace, size_t workspace_bytes,
               void *stream, xd_bfs_stats_t *stats);

/* The reference's own BFS workload. */

/* Host generator of the reference's directed fixed-degree graph (bfs.cu:354-409): rowptr[V+1],
 * col[V * degree], work_side[V] (the die that works on each vertex) and sources[num_sources].
 * The sides come from the homes of the device buffers the graph will live in: col_addr /
 * level_addr are the device addresses of col and of the level array, *_home_host host copies
 * of their xd_home_map (NULL: the address-mask prediction). Neighbour j of v is drawn as
 * xd_rand64(seed, v * degree + j) mod hot_per_side (the reference uses std::mt19937). Returns
 * XD_ERR_UNSUPPORTED when either hot pool cannot be filled (the reference exits with 2). */
int xd_bfs_ref_graph(int32_t num_vertices, int32_t degree, int32_t num_sources, int32_t dst_local_pct,
                     int32_t hot_per_side, uint64_t seed, uint64_t col_addr, const uint8_t *col_home_host,
                     uint64_t level_addr, const uint8_t *level_home_host, int32_t *rowptr, int32_t *col,
                     uint8_t *work_side, int32_t *sources);

/* Workspace bytes of xd_bfs_multi (about 24 bytes per vertex). No zeroing needed. */
size_t xd_bfs_multi_workspace_size(int32_t num_vertices);

/* Multi-source, fixed-depth top-down BFS over a directed CSR graph: level[v] = the distance
 * from the nearest source when at most max_depth, XD_BFS_UNVISITED otherwise. Sources and col
 * entries must lie in [0, V). The whole search is enqueued on `stream` (no host round trip).
 * Replaces init_dist_kernel / seed_*_kernel / luo_baseline_level_kernel /
 * luo_side_level_kernel and the fixed-depth host loops (applications/bfs/src/bfs.cu:151-308,
 * 449-491). Modes: XD_MODE_OBLIVIOUS, one frontier consumed by every workgroup; XD_MODE_AWARE,
 * one frontier per I/O die, die d consuming the vertices with work_side == d and winners
 * going to the frontier of their work side (the reference's aware run); XD_MODE_ROTATED, die
 * d consuming the other die's frontier (swapped). */
int xd_bfs_multi(const int32_t *rowptr, const int32_t *col, int32_t num_vertices, int64_t nnz,
                 const int32_t *sources, int32_t num_sources, int32_t max_depth, const uint8_t *work_side,
                 uint32_t *level, int mode, void *workspace, size_t workspace_bytes, void *stream);

/* ------------------------------------------------------------------------------------ */
/* Seeded input generators (host). Fully specified integer mixers; no libc RNG.          */
/* ------------------------------------------------------------------------------------ */

/* splitmix64 output number `index` (0-based) of the stream seeded with `seed`. */
uint64_t xd_rand64(uint64_t seed, uint64_t index);

/* out[i] = ((xd_rand64(seed, i) >> 40) * 2^-23) - 1, i.e. U[-1,1) on a 2^-23 grid. */
int xd_gen_uniform_f32(float *out, size_t n, uint64_t seed);

/* out[i] = binary16(RNE) of mean + stddev * N(0,1), Box-Muller over xd_rand64(seed, .). */
int xd_gen_normal_f16(uint16_t *out, size_t n, double mean, double stddev, uint64_t seed);

/* The reference's mix32-based inputs. mix32 is the lowbias32 finalizer of
 * applications/gemv/src/gemv_k1024_persistent_subwarp.cu:56-63.
 * xd_gen_mix32_words: out[i] = mix32((uint32_t)i ^ seed); seed 0 gives the histogram data
 * of applications/histogram/src/histogram256_sideaware.cu:331-340. */
int xd_gen_mix32_words(uint32_t *out, size_t n, uint32_t seed);

/* GEMV init_data (gemv_k1024_persistent_subwarp.cu:118-139): with h = mix32((uint32_t)i ^
 * seed), out[i] = (float)(h & 0xff) / 255.0f - 0.5f when modulus == 0, else
 * (float)((int32_t)(h % modulus) - offset) (the INTEGER_FLOAT_INPUTS variant: A uses
 * modulus 17 / offset 8 with seed, x modulus 7 / offset 3 with seed + 0x9e37). */
int xd_gen_mix32_f32(float *out, size_t n, uint32_t seed, uint32_t modulus, int32_t offset);

/* Zipf(s) over num_bins ranks as 64-bit inverse-CDF thresholds (host, fp64):
 * out[k] = floor(2^64 * sum_{r<=k} (r+1)^-s / H), out[num_bins-1] = 2^64-1. */
int xd_zipf_thresholds(uint64_t *out, uint32_t num_bins, double s);

/* Device generator: keys[i] = scramble(least k with xd_rand64(seed, i) < thresholds[k]),
 * thresholds a device copy of xd_zipf_thresholds. With scramble != 0 and num_bins a power
 * of two, rank r maps to bin ((r + 1) * 0x9E3779B1) mod num_bins (a bijection), so hot
 * ranks are spread over the bin range; otherwise bin = rank. Enqueued on `stream`. */
int xd_gen_zipf_keys(uint32_t *keys, size_t n, const uint64_t *thresholds, uint32_t num_bins,
                     uint64_t seed, int scramble, void *stream);

/* R-MAT edge e of a 2^scale-vertex graph (host): `scale` quadrant draws, most significant
 * bit first; draw l uses 32-bit word (l & 1) (low word first) of
 * xd_rand64(seed, e * ceil(scale/2) + l/2) against floor(a * 2^32), floor((a+b) * 2^32),
 * floor((a+b+c) * 2^32); quadrants c, d set the row bit and b, d the column bit. */
int xd_rmat_edge(int scale, double a, double b, double c, uint64_t seed, uint64_t e, int32_t *u,
                 int32_t *v);

/* Undirected CSR of the R-MAT graph with edge_factor * 2^scale edges (host buffers): every
 * edge (u, v), u != v, in both directions, duplicates removed, lists sorted ascending.
 * rowptr has 2^scale + 1 entries; col needs capacity >= 2 * edge_factor * 2^scale. */
int xd_rmat_csr(int scale, int edge_factor, double a, double b, double c, uint64_t seed, int32_t *rowptr,
                int32_t *col, int64_t col_capacity, int64_t *nnz_out);

#ifdef __cplusplus
}
#endif

#endif /* XDOM_H */
