// GEMV y = A.x for fp32 and fp16-with-fp32-accumulate, XCD-oblivious / aware / rotated.
//
// Reference: applications/gemv/src/gemv_k1024_persistent_subwarp.cu
//   dot_subwarp (149-161): float4 loads, per-lane partial dot over a strided K range
//   subgroup_reduce (141-147): shuffle tree over the 32 lanes of a row
//   gemv_partitioned_kernel (163-197) / gemv_baseline_kernel (199-231): row placement
//
// MI355X design: one wave64 per row at a time, 16-byte (dwordx4) loads of A, DPP wave
// reduction, and a workgroup -> row-chunk map that gives every XCD one contiguous 1/8 of the
// rows (aware) or interleaves chunks across XCDs (oblivious). x is read from global memory
// (L2-resident after the first workgroups) into registers beside the first matrix loads:
// each lane of the exact, row-home and segment-home kernels needs the same few x vectors for
// every row or segment it reduces, so staging x in LDS only put a barrier and a round trip
// ahead of the stream (cold, at 14336 x 4096 fp16: 22.5 -> 21.5 us oblivious, 21.0 -> 20.4 us
// row-home; 4096^2 fp32 segment-home 14.1 -> 13.5 us). The generic kernel, for rows that
// are not a whole number of wave-wide vectors, keeps x in LDS. No MFMA: GEMV is 0.5 (fp32) or
// 1 (fp16) flop per byte of A.
#include <hip/hip_runtime.h>


#include <algorithm>

#include "xd_common.hpp"

namespace xd {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / kWave;
constexpr int kGemvMaxLdsBytes = 64 * 1024;

__device__ __forceinline__ float dot16_f32(uint4 a, uint4 b, float acc) {
    acc = __builtin_fmaf(__uint_as_float(a.x), __uint_as_float(b.x), acc);
    acc = __builtin_fmaf(__uint_as_float(a.y), __uint_as_float(b.y), acc);
    acc = __builtin_fmaf(__uint_as_float(a.z), __uint_as_float(b.z), acc);
    acc = __builtin_fmaf(__uint_as_float(a.w), __uint_as_float(b.w), acc);
    return acc;
}

__device__ __forceinline__ float dot16_f16(uint4 a, uint4 b, float acc) {
    // v_dot2_f32_f16: fp16 products are exact in fp32; accumulation is fp32.
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a.x), __builtin_bit_cast(half2_t, b.x), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a.y), __builtin_bit_cast(half2_t, b.y), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a.z), __builtin_bit_cast(half2_t, b.z), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a.w), __builtin_bit_cast(half2_t, b.w), acc, false);
    return acc;
}

// nv = 16-byte vectors per row. U = vectors each lane keeps in flight per batch.
template <bool F16, int U>
__global__ void __launch_bounds__(kGemvThreads)
gemv_kernel(const uint4 *__restrict__ A, const uint4 *__restrict__ x, float *__restrict__ y, int M, int nv,
            int rows_per_wg, int nchunks, int mode, unsigned rot, XcdHint xh) {
    extern __shared__ uint4 xs[];
    report_xcd(xh);
    const int b = (int)blockIdx.x;
    int chunk;
    if (mode == XD_MODE_OBLIVIOUS) {
        chunk = b;
    } else {
        XcdSlot s = xcd_slot(b, (int)gridDim.x, mode, rot, xh);
        chunk = s.slice * s.per_xcd + s.rank;
    }
    if (chunk >= nchunks) return;  // whole workgroup leaves before any barrier
    const int r0 = chunk * rows_per_wg;
    const int r1 = min(M, r0 + rows_per_wg);

    for (int i = (int)threadIdx.x; i < nv; i += kGemvThreads) xs[i] = x[i];
    __syncthreads();

    const int wave = (int)threadIdx.x / kWave;
    const int lane = (int)threadIdx.x % kWave;
    for (int row = r0 + wave; row < r1; row += kGemvWaves) {
        const uint4 *arow = A + (size_t)row * (size_t)nv;
        float acc = 0.0f;
        for (int v0 = 0; v0 < nv; v0 += kWave * U) {
            uint4 a[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                int v = v0 + u * kWave + lane;
                a[u] = (v < nv) ? arow[v] : make_uint4(0, 0, 0, 0);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                int v = v0 + u * kWave + lane;
                if (v < nv) acc = F16 ? dot16_f16(a[u], xs[v], acc) : dot16_f32(a[u], xs[v], acc);
            }
        }
        acc = wave_sum_f32(acc);
        if (lane == 0) y[row] = acc;
    }
}

// Exact-width variant: each row is split into S segments of 64*CW vectors, one wave per
// segment, so every lane owns exactly CW vectors and no load needs a bounds check. The
// first row's loads are issued before the lane's CW x vectors, which stay in registers for
// every row; with DB the wave's next row is loaded while the current one is reduced (the
// launcher gives every workgroup one pass of rows, so no wave has a next row there).
// Partial sums of a split row meet in LDS.
template <bool F16, int CW, int S, bool DB>
__global__ void __launch_bounds__(kGemvThreads) __attribute__((amdgpu_waves_per_eu(4)))
gemv_exact_kernel(const uint4 *__restrict__ A, const uint4 *__restrict__ x, float *__restrict__ y, int M,
                  int rows_per_wg, int nchunks, int mode, unsigned rot, XcdHint xh) {
    report_xcd(xh);
    constexpr int nv = kWave * CW * S;
    constexpr int kRowsPerPass = kGemvWaves / S;
    __shared__ float part[kGemvWaves];
    const int b = (int)blockIdx.x;
    int chunk;
    if (mode == XD_MODE_OBLIVIOUS) {
        chunk = b;
    } else {
        XcdSlot sl = xcd_slot(b, (int)gridDim.x, mode, rot, xh);
        chunk = sl.slice * sl.per_xcd + sl.rank;
    }
    if (chunk >= nchunks) return;
    const int r0 = chunk * rows_per_wg;
    const int r1 = min(M, r0 + rows_per_wg);
    const int wave = (int)threadIdx.x / kWave;
    const int lane = (int)threadIdx.x % kWave;
    const int slot = wave / S;                  // row within a pass
    const int seg = wave % S;                   // segment of that row
    const int voff = seg * (kWave * CW) + lane; // first vector of this lane in a row

    int row = r0 + slot;
    uint4 a[CW];
    if (row < r1) {
        const uint4 *p = A + (size_t)row * nv + voff;
#pragma unroll
        for (int u = 0; u < CW; ++u) a[u] = p[u * kWave];
    }
    uint4 xr[CW];
#pragma unroll
    for (int u = 0; u < CW; ++u) xr[u] = x[voff + u * kWave];

    // Every wave runs the same number of passes so that the LDS combine barrier is uniform.
    for (int base = r0; base < r1; base += kRowsPerPass) {
        row = base + slot;
        const int next = row + kRowsPerPass;
        const bool live = row < r1;
        uint4 nb[DB ? CW : 1];
        if (DB && next < r1) {
            const uint4 *p = A + (size_t)next * nv + voff;
#pragma unroll
            for (int u = 0; u < (DB ? CW : 1); ++u) nb[u] = p[u * kWave];
        }
        float acc0 = 0.0f, acc1 = 0.0f;
        if (live) {
#pragma unroll
            for (int u = 0; u < CW; u += 2) {
                const uint4 xv0 = xr[u];
                acc0 = F16 ? dot16_f16(a[u], xv0, acc0) : dot16_f32(a[u], xv0, acc0);
                if (u + 1 < CW) {
                    const uint4 xv1 = xr[u + 1];
                    acc1 = F16 ? dot16_f16(a[u + 1], xv1, acc1) : dot16_f32(a[u + 1], xv1, acc1);
                }
            }
        }
        const float acc = wave_sum_f32(acc0 + acc1);
        if (S == 1) {
            if (live && lane == 0) y[row] = acc;
        } else {
            if (lane == 0) part[wave] = acc;
            __syncthreads();
            if (live && seg == 0 && lane == 0) {
                float t = part[wave];
#pragma unroll
                for (int k = 1; k < S; ++k) t += part[wave + k];
                y[row] = t;
            }
            __syncthreads();
        }
        if (next < r1) {
            if (DB) {
#pragma unroll
                for (int u = 0; u < (DB ? CW : 1); ++u) a[u] = nb[u];
            } else {
                const uint4 *p = A + (size_t)next * nv + voff;
#pragma unroll
                for (int u = 0; u < CW; ++u) a[u] = p[u * kWave];
            }
        }
    }
}

// Memory-home variant for rows that never straddle an 8 KiB chunk (row bytes divide 8 KiB,
// A 8 KiB aligned): each row lives on one I/O die, and the workgroups of a die take only
// the rows homed on the wanted die (aware: their own die; rotated: the other one). Rows are
// visited in groups of 8 consecutive rows; lane i of every wave evaluates the home of row
// 8g + i, and the waves of the workgroup split the group's matching rows among them.
template <bool F16, int CW>
__global__ void __launch_bounds__(kGemvThreads) __attribute__((amdgpu_waves_per_eu(4)))
gemv_rowhome_kernel(const uint4 *__restrict__ A, const uint4 *__restrict__ x, float *__restrict__ y, int M,
                    int mode, HomeMap home, XcdHint xh) {
    report_xcd(xh);
    constexpr int nv = kWave * CW;
    constexpr int kGroup = 8;
    const int b = (int)blockIdx.x;
    const int per_die = (int)gridDim.x / 2;
    const int rank = die_rank(b, xh);
    const uint32_t die = wg_die(b, xh);
    const uint32_t want = (mode == XD_MODE_AWARE) ? die : (die ^ 1u);
    const int wave = (int)threadIdx.x / kWave;
    const int lane = (int)threadIdx.x % kWave;
    uint4 xr[CW];  // the lane's x vectors, the same for every row
#pragma unroll
    for (int u = 0; u < CW; ++u) xr[u] = x[u * kWave + lane];
    const uint64_t abase = reinterpret_cast<uint64_t>(A);
    const int ngroups = (M + kGroup - 1) / kGroup;
    for (int g = rank; g < ngroups; g += per_die) {
        const int r = g * kGroup + lane;
        const bool mine = lane < kGroup && r < M && home(abase + (uint64_t)r * nv * 16) == want;
        uint64_t m = __ballot(mine);
        // drop the first `wave` matching rows, then take every kGemvWaves-th one
        for (int k = 0; k < wave && m; ++k) m &= m - 1;
        while (m) {
            const int row = g * kGroup + __builtin_ctzll(m);
            const uint4 *p = A + (size_t)row * nv + lane;
            uint4 a[CW];
#pragma unroll
            for (int u = 0; u < CW; ++u) a[u] = p[u * kWave];
            float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
            for (int u = 0; u < CW; u += 2) {
                acc0 = F16 ? dot16_f16(a[u], xr[u], acc0) : dot16_f32(a[u], xr[u], acc0);
                if (u + 1 < CW)
                    acc1 = F16 ? dot16_f16(a[u + 1], xr[u + 1], acc1) : dot16_f32(a[u + 1], xr[u + 1], acc1);
            }
            const float acc = wave_sum_f32(acc0 + acc1);
            if (lane == 0) y[row] = acc;
            for (int k = 0; k < kGemvWaves && m; ++k) m &= m - 1;
        }
    }
}

// Split-row memory-home variant for rows made of S >= 2 whole 8 KiB chunks (A 8 KiB
// aligned). Segment j (bytes [8 KiB j, 8 KiB (j+1)) of A) is part j % S of row j / S and is
// homed on one I/O die; the waves of a die take the segments homed on the wanted die. A
// segment's partial is computed exactly as the exact-width kernel's wave for that segment
// computes it (8 vectors per lane, same lane -> vector map, same reduction), and the row's
// partials meet through memory-side atomics on the workspace:
//   S == 2 (PAIR): each arrival swaps a 64-bit word (segment + 1) << 32 | bits(partial) into
//     the row's word; the arrival that gets its partner's word back writes y = p0 + p1
//     (fp addition is commutative, so the order of arrival does not change the bits) and
//     clears the word (in the kernel below).
//   S > 2 (seg_meet): each arrival deposits its partial in slot j with a returning swap, then
//     takes a ticket on the row's counter; the last of the S arrivals swaps the slots back
//     out, adds them in segment order, writes y and clears the counter.
// Both orders equal the exact kernel's LDS combine order, so both kernels give the same bits
// for S = 2 and 4. The row words / counters must be zero when the call starts; every call
// leaves them zero.
__device__ __forceinline__ void seg_meet(float part, int j, int row, int seg, int S, float *__restrict__ y,
                                         uint32_t *__restrict__ cnt, uint32_t *__restrict__ slot) {
    const uint32_t old = atomicExch(&slot[j], __float_as_uint(part));
    // consuming the returned value makes the ticket wait until the deposit is done
    asm volatile("" ::"v"(old));
    const uint32_t t = atomicAdd(&cnt[row], 1u);
    if (t == (uint32_t)(S - 1)) {
        float sum = 0.0f;
        for (int s = 0; s < S; ++s) {
            // a swap is a read-modify-write executed at the memory-side atomic unit, like
            // the deposit it reads (an idempotent OR could become a plain load)
            const float v = (s == seg) ? part : __uint_as_float(atomicExch(&slot[(size_t)row * S + s], 0u));
            sum = (s == 0) ? v : sum + v;
        }
        y[row] = sum;
        atomicExch(&cnt[row], 0u);
    }
}

// Workgroup w of a die visits groups w, w + W, w + 2W, ... of 8 consecutive segments (W =
// workgroups per die); the lanes of every wave evaluate the homes of the next 8 such groups
// at once (one page-map load per lane), and each group's wanted segments are dealt to the 4
// waves in turn. S == 2: a segment's exchange is issued after its reduction and its returned
// word is used only after the wave's next segment's loads are out, so the round trip overlaps
// them (the vector-memory counter is in order: the swap is older than those loads, and the
// wait for it leaves them in flight). 4096 x 4096 fp32 cold: 13.67 -> 13.48 us.
template <bool F16, bool PAIR>
__global__ void __launch_bounds__(kGemvThreads) __attribute__((amdgpu_waves_per_eu(4)))
gemv_seghome_kernel(const uint4 *__restrict__ A, const uint4 *__restrict__ x, float *__restrict__ y, int M, int S,
                    int mode, HomeMap home, uint32_t *__restrict__ cnt, uint32_t *__restrict__ slot, XcdHint xh) {
    report_xcd(xh);
    constexpr int CW = 8;
    constexpr int kSegVec = kWave * CW;  // 512 vectors = 8 KiB
    constexpr int kGroup = 8;
    const int b = (int)blockIdx.x;
    const int per_die = (int)gridDim.x / 2;
    const int rank = die_rank(b, xh);
    const uint32_t die = wg_die(b, xh);
    const uint32_t want = (mode == XD_MODE_AWARE) ? die : (die ^ 1u);
    const int wave = (int)threadIdx.x / kWave;
    const int lane = (int)threadIdx.x % kWave;
    const uint64_t abase = reinterpret_cast<uint64_t>(A);
    const int nseg = M * S;
    const int ngroups = (nseg + kGroup - 1) / kGroup;
    // segment j: its matrix vectors and the matching x vectors (segment j % S of x) loaded
    // together, then the previous segment's meet settled, then j reduced and its meet issued.
    auto seg_loads = [&](int j, uint4 (&a)[CW], uint4 (&xv)[CW]) {
        const int seg = j % S;
        const uint4 *p = A + (size_t)j * kSegVec + lane;
        const uint4 *xp = x + (size_t)seg * kSegVec + lane;
#pragma unroll
        for (int u = 0; u < CW; ++u) a[u] = p[u * kWave];
#pragma unroll
        for (int u = 0; u < CW; ++u) xv[u] = xp[u * kWave];
    };
    auto seg_sum = [&](const uint4 (&a)[CW], const uint4 (&xv)[CW]) {
        float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
        for (int u = 0; u < CW; u += 2) {
            acc0 = F16 ? dot16_f16(a[u], xv[u], acc0) : dot16_f32(a[u], xv[u], acc0);
            acc1 = F16 ? dot16_f16(a[u + 1], xv[u + 1], acc1) : dot16_f32(a[u + 1], xv[u + 1], acc1);
        }
        return wave_sum_f32(acc0 + acc1);
    };
    unsigned long long *pw = reinterpret_cast<unsigned long long *>(cnt);
    int prow = -1;
    float ppart = 0.0f;
    unsigned long long pold = 0ull;
    auto settle = [&]() {
        if (lane == 0 && prow >= 0 && pold != 0ull) {
            y[prow] = ppart + __uint_as_float((uint32_t)pold);
            atomicExch(&pw[prow], 0ull);
        }
    };
    // lane l evaluates segment l % 8 of the l / 8-th of the next 8 groups this workgroup visits
    for (int g0 = rank; g0 < ngroups; g0 += kGroup * per_die) {
        const int gl = g0 + (lane / kGroup) * per_die;
        const int jl = gl * kGroup + lane % kGroup;
        const bool wanted = gl < ngroups && jl < nseg && home(abase + (uint64_t)jl * kHomeChunk) == want;
        const uint64_t all = __ballot(wanted);
        for (int q = 0; q < kGroup; ++q) {
            const int g = g0 + q * per_die;
            if (g >= ngroups) break;
            uint64_t m = (all >> (q * kGroup)) & 0xffull;
            for (int k = 0; k < wave && m; ++k) m &= m - 1;
            while (m) {
                const int j = g * kGroup + __builtin_ctzll(m);
                uint4 a[CW], xv[CW];
                seg_loads(j, a, xv);
                if (PAIR) {
                    settle();
                    const float part = seg_sum(a, xv);
                    const int row = j / S;
                    if (lane == 0) {
                        const unsigned long long word =
                            ((unsigned long long)(j - row * S + 1) << 32) | (unsigned long long)__float_as_uint(part);
                        pold = atomicExch(&pw[row], word);
                    }
                    prow = row;
                    ppart = part;
                } else {
                    const float part = seg_sum(a, xv);
                    const int row = j / S;
                    if (lane == 0) seg_meet(part, j, row, j - row * S, S, y, cnt, slot);
                }
                for (int k = 0; k < kGemvWaves && m; ++k) m &= m - 1;
            }
        }
    }
    if (PAIR) settle();
}

// Rows that straddle 8 KiB chunks without being whole chunks (the fp16 down projection's
// 28 KiB rows) take the exact kernel in every mode, the aware one with each XCD on one
// contiguous eighth of the rows. A chunk-home route for them (each 8 KiB chunk reduced on its
// home die, the pieces of a row added by a second launch) ran 15.7 + 3.7 us warm and 23.2 +
// 4.1 us cold at 4096 x 14336 fp16, against 17.6 / 20.6 us for the contiguous eighths and
// 17.6 / 21.2 us oblivious: the second launch and the split rows cost more than the near
// chunks save, and cold there is nothing to save.

static int seg_per_row(int K, int elem_bytes) {
    const size_t row_bytes = (size_t)K * (size_t)elem_bytes;
    if (row_bytes % kHomeChunk != 0) return 0;
    const size_t S = row_bytes / kHomeChunk;
    return (S >= 2 && S * kHomeChunk <= (size_t)kGemvMaxLdsBytes) ? (int)S : 0;
}

static int rows_per_workgroup(int M, int nv) {
    // (the generic kernel, rows of a length that is not a multiple of 64 vectors) Aim for
    // >= 4 workgroups per CU on 256 CUs and one row per wave for long rows.
    int rpw = kGemvWaves;
    while ((long long)M / (rpw * 2) >= 1024 && nv * 16 * rpw * 2 <= 256 * 1024) rpw *= 2;
    return rpw;
}

template <bool F16>
static int launch_gemv(const void *A, const void *x, float *y, int M, int K, int mode, const uint8_t *home_attr,
                       void *workspace, size_t workspace_bytes, void *stream) {
    const int per_vec = F16 ? 8 : 4;
    XD_REQUIRE(A != nullptr && x != nullptr && y != nullptr, "gemv: NULL pointer");
    XD_REQUIRE(M > 0 && K > 0, "gemv: M and K must be positive");
    XD_REQUIRE(K % per_vec == 0, F16 ? "gemv_f16f32: K must be a multiple of 8" : "gemv_f32: K must be a multiple of 4");
    XD_REQUIRE(aligned16(A) && aligned16(x), "gemv: A and x must be 16-byte aligned");
    XD_REQUIRE(mode >= XD_MODE_OBLIVIOUS && mode <= XD_MODE_ROTATED, "gemv: bad mode");
    const int nv = K / per_vec;
    const size_t lds = (size_t)nv * 16;
    if (lds > (size_t)kGemvMaxLdsBytes) return fail(XD_ERR_UNSUPPORTED, "gemv: K too large for the LDS-staged x");
    const int rpw = rows_per_workgroup(M, nv);
    const int nchunks = (M + rpw - 1) / rpw;
    const int grid = ((nchunks + kNumXcd - 1) / kNumXcd) * kNumXcd;
    // rotated: slice s on XCD (s + rot) mod 8 with rot in [1, 8), never the identity placement
    unsigned rot = mode == XD_MODE_ROTATED ? next_rotation(1) % kNumXcd : 0u;
    if (mode == XD_MODE_ROTATED && rot == 0) rot = 1;
    hipStream_t s = (hipStream_t)stream;
    const XcdHint xh = xcd_hint(s);
    const uint4 *A4 = reinterpret_cast<const uint4 *>(A);
    const uint4 *x4 = reinterpret_cast<const uint4 *>(x);
    bool done = false;
    // Memory-home routing of 8 KiB row segments when rows are whole multiples of 8 KiB.
    const int S = seg_per_row(K, F16 ? 2 : 4);
    if (mode != XD_MODE_OBLIVIOUS && S > 0 && (reinterpret_cast<uintptr_t>(A) % kHomeChunk) == 0 && workspace &&
        workspace_bytes >= (size_t)M * (size_t)(S + 1) * 4 && (reinterpret_cast<uintptr_t>(workspace) % 8) == 0) {
        const HomeMap home{home_attr, reinterpret_cast<uint64_t>(A) / kHomePage, home_mask()};
        uint32_t *cnt = reinterpret_cast<uint32_t *>(workspace);
        uint32_t *slot = cnt + M;
        const long long nseg = (long long)M * S;
        // one workgroup per 8 segments (two groups of 8 per workgroup on average, about one
        // wanted segment per wave per group); measured best among 4, 8 and 16 per workgroup
        long long sgrid = (nseg + 7) / 8;
        sgrid = (sgrid + kNumXcd - 1) / kNumXcd * kNumXcd;
        if (sgrid > (1LL << 30)) return fail(XD_ERR_UNSUPPORTED, "gemv: matrix too large for the split-row route");
        if (S == 2)
            launch("gemv_seghome_kernel", gemv_seghome_kernel<F16, true>, dim3((unsigned)sgrid), dim3(kGemvThreads), 0, s, A4, x4,
                               y, M, S, mode, home, cnt, slot, xh);
        else
            launch("gemv_seghome_kernel", gemv_seghome_kernel<F16, false>, dim3((unsigned)sgrid), dim3(kGemvThreads), 0, s, A4,
                               x4, y, M, S, mode, home, cnt, slot, xh);
        done = true;
    }
    // Memory-home routing when every row sits inside one 8 KiB chunk.
    const size_t row_bytes = (size_t)nv * 16;
    if (!done && mode != XD_MODE_OBLIVIOUS && kHomeChunk % row_bytes == 0 &&
        (reinterpret_cast<uintptr_t>(A) % kHomeChunk) == 0 && nv % kWave == 0) {
        const int CW = nv / kWave;
        const HomeMap home{home_attr, reinterpret_cast<uint64_t>(A) / kHomePage, home_mask()};
        // two groups of 8 rows per workgroup on average
        int hgrid = ((M + 15) / 16 + kNumXcd - 1) / kNumXcd * kNumXcd;
        if (hgrid < kNumXcd) hgrid = kNumXcd;
        done = true;
#define XD_GEMV_HOME(CC)                                                                                       \
    if (CW == CC) {                                                                                           \
        launch("gemv_rowhome_kernel", gemv_rowhome_kernel<F16, CC>, dim3(hgrid), dim3(kGemvThreads), 0, s, A4, x4, y, M, \
                           mode, home, xh);                                                                        \
    } else
        XD_GEMV_HOME(1)
        XD_GEMV_HOME(2)
        XD_GEMV_HOME(4)
        XD_GEMV_HOME(8)
        { done = false; }
#undef XD_GEMV_HOME
    }
    if (!done && nv % kWave == 0) {
        // smallest split S (1, 2, 4) with at most 8 vectors per lane per wave
        const int C = nv / kWave;
        int S = 1;
        while (S < kGemvWaves && (C % (S * 2) == 0) && C / S > 8) S *= 2;
        const int CW = C / S;
        // one pass of kGemvWaves / S rows per workgroup: the dispatcher refills CUs as
        // workgroups finish, which beat rows double-buffered over several passes (2 or 4 per
        // workgroup) from HBM by 4-12 % at 4096^2 fp32 and both fp16 decode shapes
        const int erpw = kGemvWaves / S;
        const int enchunks = (M + erpw - 1) / erpw;
        const int egrid = ((enchunks + kNumXcd - 1) / kNumXcd) * kNumXcd;
        // No home route applies here (rows straddle 8 KiB chunks, or no workspace or page
        // alignment): the aware call keeps the round robin, which from HBM beat giving each
        // XCD a contiguous eighth of the rows by 4 % at fp16 4096 x 14336 (level warm);
        // rotated keeps the rotated eighths as its control.
        const int emode = mode == XD_MODE_AWARE ? XD_MODE_OBLIVIOUS : mode;
        done = true;
#define XD_GEMV_EXACT(CC, SS, DBB)                                                                        \
    if (CW == CC && S == SS) {                                                                          \
        launch("gemv_exact_kernel", gemv_exact_kernel<F16, CC, SS, DBB>, dim3(egrid), dim3(kGemvThreads), 0, s, A4, \
                           x4, y, M, erpw, enchunks, emode, rot, xh);                                         \
    } else
        XD_GEMV_EXACT(1, 1, true)
        XD_GEMV_EXACT(2, 1, true)
        XD_GEMV_EXACT(3, 1, true)
        XD_GEMV_EXACT(4, 1, true)
        XD_GEMV_EXACT(5, 1, true)
        XD_GEMV_EXACT(6, 1, true)
        XD_GEMV_EXACT(7, 1, true)
        XD_GEMV_EXACT(8, 1, true)
        XD_GEMV_EXACT(5, 2, true)
        XD_GEMV_EXACT(6, 2, true)
        XD_GEMV_EXACT(7, 2, true)
        XD_GEMV_EXACT(8, 2, true)
        XD_GEMV_EXACT(5, 4, true)
        XD_GEMV_EXACT(6, 4, true)
        XD_GEMV_EXACT(7, 4, true)
        XD_GEMV_EXACT(8, 4, true)
        { done = false; }
#undef XD_GEMV_EXACT
    }
    if (!done) {
        if (nv >= kWave * 16) {
            launch("gemv_kernel", gemv_kernel<F16, 16>, dim3(grid), dim3(kGemvThreads), lds, s, A4, x4, y, M, nv, rpw,
                               nchunks, mode, rot, xh);
        } else {
            launch("gemv_kernel", gemv_kernel<F16, 8>, dim3(grid), dim3(kGemvThreads), lds, s, A4, x4, y, M, nv, rpw,
                               nchunks, mode, rot, xh);
        }
    }
    return launch_status("gemv_kernel");
}

}  // namespace xd

using namespace xd;

extern "C" {

size_t xd_gemv_workspace_size(int M, int K, int elem_bytes) {
    if (M <= 0 || K <= 0 || (elem_bytes != 2 && elem_bytes != 4)) return 0;
    const int S = seg_per_row(K, elem_bytes);
    return S > 0 ? (size_t)M * (size_t)(S + 1) * 4 : 0;
}

int xd_gemv_f32(const float *A, const float *x, float *y, int M, int K, int mode, const uint8_t *home_attr,
                void *workspace, size_t workspace_bytes, void *stream) {
    return launch_gemv<false>(A, x, y, M, K, mode, home_attr, workspace, workspace_bytes, stream);
}

int xd_gemv_f16f32(const uint16_t *W, const uint16_t *x, float *y, int M, int K, int mode, const uint8_t *home_attr,
                   void *workspace, size_t workspace_bytes, void *stream) {
    return launch_gemv<true>(W, x, y, M, K, mode, home_attr, workspace, workspace_bytes, stream);
}

}  // extern "C"
