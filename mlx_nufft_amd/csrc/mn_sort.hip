// Stable bin sort and subproblem tables.
//
// The bin sort is an LSD radix sort over digits of the bin key (at most 8
// bits, the key split evenly over the passes). Each
// pass is (1) a per-tile digit histogram, (2) an exclusive scan of each
// digit's counts over the tiles (the scatter adds the digit bases, the scan
// of the 256 digit totals), (3) a stable scatter in which every tile
// ranks its elements in index order with wave ballots (64-lane match on the
// 8 digit bits) and LDS counters. LSD radix passes are stable, so the final
// permutation equals numpy's argsort(key, kind="stable")
// (ref: nd.py:314, nd.py:175, gpu_t3.py:490-492).
//
// The subproblem table replaces the reference's host-side construction
// (ref: nd.py:347-372) with three device kernels and one 8-byte read-back.
#include <mutex>

#include "mn_common.h"

namespace mn {
namespace {

constexpr int RS_THREADS = 256;
// 8192-element tiles: twice the digit-run length of 4096-element ones, so
// fewer partial cache lines at the run ends (measured 9 % faster per set of
// passes at 2e7 keys; 12288 spills registers)
constexpr int RS_ITEMS = 32;
constexpr int RS_TILE = RS_THREADS * RS_ITEMS;  // 8192 elements per tile
constexpr int RS_RADIX = 256;

constexpr int SC_THREADS = 256;
constexpr int SC_ITEMS = 8;
constexpr int SC_TILE = SC_THREADS * SC_ITEMS;  // 2048 elements per scan tile

// ---------------------------------------------------------------- scan ----

__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        uint32_t t = __shfl_up(v, o, 64);
        if (lane >= o) v += t;
    }
    return v;
}

// Exclusive scan of the thread totals of one block of NT threads (NT a
// multiple of 64); returns the exclusive prefix of this thread and writes
// the block total to *total.
template <int NT>
__device__ __forceinline__ uint32_t block_excl_scan_n(uint32_t v, uint32_t *total) {
    __shared__ uint32_t wsum[NT / 64];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    uint32_t inc = wave_incl_scan(v);
    if (lane == 63) wsum[wv] = inc;
    __syncthreads();
    uint32_t off = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) {
        uint32_t s = wsum[w];
        if (w < wv) off += s;
        tot += s;
    }
    __syncthreads();
    *total = tot;
    return off + inc - v;
}

__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t *total) {
    return block_excl_scan_n<SC_THREADS>(v, total);
}

// The scatter takes a tile with 512 threads, 16 elements each: 104 VGPRs and
// four waves per SIMD (256 threads with 32 elements each needed 180 VGPRs,
// two waves per SIMD, and took 0.72 ms for three passes at 2e7 keys and
// three payload columns against 0.68; 1024 threads with 8 each took 0.79)
constexpr int ST_THREADS = 512;
constexpr int ST_ITEMS = RS_TILE / ST_THREADS;

__global__ void k_tile_reduce(const uint32_t *__restrict__ d, int64_t n,
                              uint32_t *__restrict__ partials) {
    int64_t base = (int64_t)blockIdx.x * SC_TILE + (int64_t)threadIdx.x * SC_ITEMS;
    uint32_t s = 0;
#pragma unroll
    for (int i = 0; i < SC_ITEMS; ++i)
        if (base + i < n) s += d[base + i];
    uint32_t tot;
    block_excl_scan(s, &tot);
    if (threadIdx.x == 0) partials[blockIdx.x] = tot;
}

// Exclusive scan of one tile in place, offset by partials[blockIdx.x] when
// partials is non-NULL.
__global__ void k_tile_scan(uint32_t *__restrict__ d, int64_t n,
                            const uint32_t *__restrict__ partials) {
    int64_t base = (int64_t)blockIdx.x * SC_TILE + (int64_t)threadIdx.x * SC_ITEMS;
    uint32_t v[SC_ITEMS];
    uint32_t s = 0;
#pragma unroll
    for (int i = 0; i < SC_ITEMS; ++i) {
        v[i] = (base + i < n) ? d[base + i] : 0u;
        s += v[i];
    }
    uint32_t tot;
    uint32_t run = block_excl_scan(s, &tot);
    if (partials) run += partials[blockIdx.x];
#pragma unroll
    for (int i = 0; i < SC_ITEMS; ++i) {
        if (base + i < n) d[base + i] = run;
        run += v[i];
    }
}

// ---------------------------------------------------------- radix sort ----

// The pass's digit: width bits of the masked key from shift on, dmask =
// 2^width - 1 (width <= 8).
__device__ __forceinline__ uint32_t digit_of(uint32_t k, uint32_t kmask, int shift,
                                             uint32_t dmask) {
    return ((k & kmask) >> shift) & dmask;
}

// Row d of the digit-major histogram (hist[d * nblk + t], t = tile) scanned
// over the tiles in place (exclusive), one workgroup per digit; totals[d] =
// the digit's count. The scatter turns the totals into digit bases itself,
// so a pass needs this one launch instead of a multi-level scan of the
// whole matrix. (A tile-major matrix was measured: its histogram writes
// were 3.6 us faster per pass, its strided scan 7 us slower.)
constexpr int DS_ITEMS = 16;
__global__ __launch_bounds__(SC_THREADS) void k_digit_scan(uint32_t *__restrict__ hist,
                                                           int64_t nblk,
                                                           uint32_t *__restrict__ totals) {
    uint32_t *row = hist + (int64_t)blockIdx.x * nblk;
    uint32_t carry = 0;
    for (int64_t b0 = 0; b0 < nblk; b0 += SC_THREADS * DS_ITEMS) {
        const int64_t i0 = b0 + (int64_t)threadIdx.x * DS_ITEMS;
        uint32_t v[DS_ITEMS], s = 0;
#pragma unroll
        for (int i = 0; i < DS_ITEMS; ++i) {
            v[i] = i0 + i < nblk ? row[i0 + i] : 0u;
            s += v[i];
        }
        uint32_t tot;
        uint32_t run = block_excl_scan(s, &tot) + carry;
#pragma unroll
        for (int i = 0; i < DS_ITEMS; ++i) {
            if (i0 + i < nblk) row[i0 + i] = run;
            run += v[i];
        }
        carry += tot;
    }
    if (threadIdx.x == 0) totals[blockIdx.x] = carry;
}

// Per-tile digit counts. Each wave counts into its own LDS histogram (fewer
// same-address atomics than one shared by the workgroup); whole tiles of a
// 16-byte aligned key array are read as 16-byte vectors.
__global__ __launch_bounds__(RS_THREADS) void k_radix_hist(const uint32_t *__restrict__ keys,
                                                           int64_t P, int shift, uint32_t kmask,
                                                           uint32_t dmask,
                                                           uint32_t *__restrict__ hist,
                                                           int64_t nblk) {
    static_assert(RS_THREADS == RS_RADIX, "a thread per digit");
    constexpr int NW = RS_THREADS / 64;
    __shared__ uint32_t h[NW][RS_RADIX];
    const int tid = threadIdx.x, wv = tid >> 6;
#pragma unroll
    for (int w = 0; w < NW; ++w) h[w][tid] = 0;
    __syncthreads();
    // tiles XCD-contiguous, as in the scatter: a digit row's entries of
    // neighbouring tiles then leave one L2 as whole lines
    const int64_t tile = xcd_remap(blockIdx.x, nblk);
    const int64_t base = tile * RS_TILE;
    const bool vec = base + RS_TILE <= P && (reinterpret_cast<uintptr_t>(keys) & 15) == 0;
    if (vec) {
        constexpr int NV = RS_ITEMS / 4;
        const uint4 *k4 = reinterpret_cast<const uint4 *>(keys + base);
        uint4 kv[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) kv[i] = k4[i * RS_THREADS + tid];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            atomicAdd(&h[wv][digit_of(kv[i].x, kmask, shift, dmask)], 1u);
            atomicAdd(&h[wv][digit_of(kv[i].y, kmask, shift, dmask)], 1u);
            atomicAdd(&h[wv][digit_of(kv[i].z, kmask, shift, dmask)], 1u);
            atomicAdd(&h[wv][digit_of(kv[i].w, kmask, shift, dmask)], 1u);
        }
    } else {
        uint32_t kv[RS_ITEMS];
#pragma unroll
        for (int i = 0; i < RS_ITEMS; ++i) {
            const int64_t idx = base + (int64_t)i * RS_THREADS + tid;
            kv[i] = idx < P ? keys[idx] : 0u;
        }
#pragma unroll
        for (int i = 0; i < RS_ITEMS; ++i) {
            const int64_t idx = base + (int64_t)i * RS_THREADS + tid;
            if (idx < P) atomicAdd(&h[wv][digit_of(kv[i], kmask, shift, dmask)], 1u);
        }
    }
    __syncthreads();
    // rows of the pass's 2^width digits only; the digit scan reads no others
    if (tid <= (int)dmask) {
        uint32_t s = 0;
#pragma unroll
        for (int w = 0; w < NW; ++w) s += h[w][tid];
        hist[(int64_t)tid * nblk + tile] = s;
    }
}

struct SortCols {
    const uint32_t *in[MN_SORT_MAX_COLS];
    uint32_t *out[MN_SORT_MAX_COLS];
};

// Stable scatter of one 8192-element tile: the key, its value (the caller
// index; implicit on the first pass) and up to MN_SORT_MAX_COLS payload
// columns.
//  1. Rank: wave w owns the tile's elements [1024w, 1024w + 1024) and visits
//     them in 16 rounds of 64 consecutive elements; lanes with equal digits
//     find each other with a ballot match and a wave-private LDS counter per
//     digit gives the count of the wave's earlier elements with that digit.
//     No barrier is needed inside a wave (its LDS accesses stay in order).
//  2. One scan over the 8 x 256 wave counters gives each (wave, digit) its
//     start in the tile-local sorted order; an element's slot is that start
//     plus its rank. Index order is kept, so the pass is stable.
//  3. Every column goes through LDS: written at the slots, read back in slot
//     order and stored at gbase[d] + slot - lstart[d], so consecutive lanes
//     store consecutive addresses inside each digit run.
// Tiles are mapped XCD-contiguously, so the runs that adjacent tiles write
// for one digit meet in the same L2 and leave as whole lines.
__global__ __launch_bounds__(ST_THREADS) void k_radix_scatter(
    const uint32_t *__restrict__ kin, const uint32_t *__restrict__ vin, int64_t P, int shift,
    uint32_t kmask, uint32_t dmask, const uint32_t *__restrict__ offs, const uint32_t *__restrict__ totals,
    int64_t nblk, uint32_t *__restrict__ kout, uint32_t *__restrict__ vout, int ncols,
    SortCols cols) {
    static_assert(ST_THREADS >= RS_RADIX, "a thread per digit");
    constexpr int NWV = ST_THREADS / 64;
    __shared__ uint32_t gbase[RS_RADIX];
    __shared__ uint32_t lstart[RS_RADIX];
    __shared__ uint32_t wcnt[NWV][RS_RADIX];
    __shared__ uint32_t stage[RS_TILE];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int64_t tile = xcd_remap(blockIdx.x, nblk);
    const int64_t base = tile * RS_TILE;
    const int nvalid = (int)((P - base) < RS_TILE ? (P - base) : RS_TILE);
    const bool dt = tid < RS_RADIX;  // a thread per digit
    const bool du = tid <= (int)dmask;  // a digit of this pass (scanned over the tiles)
    {
        // the digit's base (all smaller digits) plus the tiles before this one
        const uint32_t toff = du ? offs[(int64_t)tid * nblk + tile] : 0u;
        uint32_t all;
        const uint32_t ex = block_excl_scan_n<ST_THREADS>(du ? totals[tid] : 0u, &all);
        if (dt) gbase[tid] = ex + toff;
    }
#pragma unroll
    for (int w = 0; w < NWV; ++w)
        if (dt) wcnt[w][tid] = 0;
    __syncthreads();
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    uint32_t kv[ST_ITEMS], rk[ST_ITEMS];
    const int wbase = wv * (RS_TILE / NWV);
    // all key loads first: one memory latency per tile, not one per round
#pragma unroll
    for (int r = 0; r < ST_ITEMS; ++r) {
        const int q = wbase + r * 64 + lane;
        kv[r] = q < nvalid ? kin[base + q] : 0u;
    }
#pragma unroll
    for (int r = 0; r < ST_ITEMS; ++r) {
        const int q = wbase + r * 64 + lane;
        const bool valid = q < nvalid;
        const uint32_t k = kv[r];
        const uint32_t dg = digit_of(k, kmask, shift, dmask);
        uint64_t peers = __ballot(valid);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const bool bit = (dg >> b) & 1u;
            const uint64_t bal = __ballot(bit);
            peers &= bit ? bal : ~bal;
        }
        const uint32_t rank = (uint32_t)__popcll(peers & lt_mask);
        const uint32_t before = valid ? wcnt[wv][dg] : 0u;
        if (valid && rank == 0) wcnt[wv][dg] = before + (uint32_t)__popcll(peers);
        rk[r] = valid ? ((dg << 16) | (before + rank)) : 0xFFFFFFFFu;
    }
    __syncthreads();
    // Tile-local starts: digit-major over (digit, wave).
    {
        uint32_t c[NWV], s = 0;
#pragma unroll
        for (int w = 0; w < NWV; ++w) {
            c[w] = dt ? wcnt[w][tid] : 0u;
            s += c[w];
        }
        uint32_t tot;
        const uint32_t ex = block_excl_scan_n<ST_THREADS>(s, &tot);
        if (dt) {
            lstart[tid] = ex;
            uint32_t run = ex;
#pragma unroll
            for (int w = 0; w < NWV; ++w) {
                wcnt[w][tid] = run;
                run += c[w];
            }
        }
    }
    __syncthreads();
    int slot[ST_ITEMS];
#pragma unroll
    for (int r = 0; r < ST_ITEMS; ++r)
        slot[r] = rk[r] == 0xFFFFFFFFu ? -1 : (int)(wcnt[wv][rk[r] >> 16] + (rk[r] & 0xFFFFu));
    // Keys: stage, then derive each slot's destination from its digit.
#pragma unroll
    for (int r = 0; r < ST_ITEMS; ++r)
        if (slot[r] >= 0) stage[slot[r]] = kv[r];
    __syncthreads();
    uint32_t dst[ST_ITEMS];
#pragma unroll
    for (int r = 0; r < ST_ITEMS; ++r) {
        const int q = r * ST_THREADS + tid;
        dst[r] = 0;
        if (q < nvalid) {
            const uint32_t k = stage[q];
            const uint32_t d = digit_of(k, kmask, shift, dmask);
            dst[r] = gbase[d] + (uint32_t)q - lstart[d];
            kout[dst[r]] = k;
        }
    }
    __syncthreads();
    // Values and payload columns, one LDS round trip each; the next
    // column's loads are issued before the current one is written out.
    uint32_t cur[ST_ITEMS];
#pragma unroll
    for (int r = 0; r < ST_ITEMS; ++r) {
        const int64_t idx = base + wbase + r * 64 + lane;
        cur[r] = slot[r] >= 0 ? (vin ? vin[idx] : (uint32_t)idx) : 0u;
    }
    for (int c = -1; c < ncols; ++c) {
        uint32_t *out = c < 0 ? vout : cols.out[c];
#pragma unroll
        for (int r = 0; r < ST_ITEMS; ++r)
            if (slot[r] >= 0) stage[slot[r]] = cur[r];
        __syncthreads();
        if (c + 1 < ncols) {
            const uint32_t *src = cols.in[c + 1];
#pragma unroll
            for (int r = 0; r < ST_ITEMS; ++r) {
                const int64_t idx = base + wbase + r * 64 + lane;
                cur[r] = slot[r] >= 0 ? src[idx] : 0u;
            }
        }
#pragma unroll
        for (int r = 0; r < ST_ITEMS; ++r) {
            const int q = r * ST_THREADS + tid;
            if (q < nvalid) out[dst[r]] = stage[q];
        }
        __syncthreads();
    }
}

// starts[k] = first sorted index whose key (masked by kmask) is >= k, for k
// in [0, K]: sorted position j (j in [0, P]) writes j for every key in
// (key[j-1], key[j]] (from 0 for j = 0, up to K for j = P). A thread takes
// KS_ITEMS positions 256 apart, so every load is coalesced and a wave keeps
// 2 KS_ITEMS loads in flight (one position per thread left the kernel
// waiting on memory latency). Short ranges are written by their lane; long
// ones (sparse or clustered points) by the whole wave, 64 consecutive
// entries per store.
constexpr int KS_THREADS = 256;
constexpr int KS_ITEMS = 8;
__global__ __launch_bounds__(KS_THREADS) void k_key_starts(const uint32_t *__restrict__ key,
                                                           int64_t P, int64_t K, uint32_t kmask,
                                                           int32_t *__restrict__ starts) {
    const int64_t j0 = (int64_t)blockIdx.x * (KS_THREADS * KS_ITEMS) + threadIdx.x;
    const int lane = threadIdx.x & 63;
    int64_t lo[KS_ITEMS], hi[KS_ITEMS];  // inclusive key range to fill with j
#pragma unroll
    for (int i = 0; i < KS_ITEMS; ++i) {
        const int64_t j = j0 + (int64_t)i * KS_THREADS;
        const uint32_t kp = (j >= 1 && j <= P) ? key[j - 1] : 0u;
        const uint32_t kj = j < P ? key[j] : 0u;
        lo[i] = j == 0 ? 0 : (int64_t)(kp & kmask) + 1;
        hi[i] = j < P ? (int64_t)(kj & kmask) : (j == P ? K : -1);
    }
#pragma unroll
    for (int i = 0; i < KS_ITEMS; ++i) {
        const int32_t j = (int32_t)(j0 + (int64_t)i * KS_THREADS);
        const bool big = hi[i] - lo[i] >= 16;
        if (!big)
            for (int64_t k = lo[i]; k <= hi[i]; ++k) starts[k] = j;
        uint64_t todo = __ballot(big);
        while (todo) {
            const int src = __ffsll((unsigned long long)todo) - 1;
            todo &= todo - 1;
            const int64_t blo = __shfl(lo[i], src, 64), bhi = __shfl(hi[i], src, 64);
            const int32_t v = __shfl(j, src, 64);
            for (int64_t k = blo + lane; k <= bhi; k += 64) starts[k] = v;
        }
    }
}

// --------------------------------------------------------- subproblems ----

__global__ void k_bin_bounds(const uint32_t *__restrict__ skey, int64_t P, int64_t nbins,
                             int32_t *__restrict__ bstart, int32_t *__restrict__ bend) {
    int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= P) return;
    uint32_t k = skey[j];
    if ((int64_t)k >= nbins) return;  // keys come from setpts and are < nbins
    if (j == 0 || skey[j - 1] != k) bstart[k] = (int32_t)j;
    if (j == P - 1 || skey[j + 1] != k) bend[k] = (int32_t)(j + 1);
}

__global__ void k_bin_nsub(const int32_t *__restrict__ bstart, const int32_t *__restrict__ bend,
                           int64_t nbins, int32_t msub, uint32_t *__restrict__ nsub) {
    int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b > nbins) return;
    if (b == nbins) {
        nsub[b] = 0;
        return;
    }
    int32_t c = bend[b] - bstart[b];
    nsub[b] = (uint32_t)((c + msub - 1) / msub);
}

__global__ void k_sub_fill(const int32_t *__restrict__ bstart, const int32_t *__restrict__ bend,
                           const uint32_t *__restrict__ soff, int64_t nbins, int32_t msub,
                           int32_t *__restrict__ info) {
    int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nbins) return;
    int32_t s0 = bstart[b], c = bend[b] - s0;
    uint32_t row = soff[b];
    for (int32_t o = 0; o < c; o += msub, ++row) {
        info[3 * (int64_t)row + 0] = (int32_t)b;
        info[3 * (int64_t)row + 1] = s0 + o;
        info[3 * (int64_t)row + 2] = (c - o < msub) ? (c - o) : msub;
    }
}

inline unsigned blocks_for(int64_t n, int t) { return (unsigned)((n + t - 1) / t); }

inline int64_t align_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

}  // namespace

int64_t scan_partials_elems(int64_t n) {
    int64_t tot = 0;
    while (n > SC_TILE) {
        n = (n + SC_TILE - 1) / SC_TILE;
        tot += n;
    }
    return tot + 1;
}

int scan_exclusive_u32(uint32_t *data, int64_t n, uint32_t *partials, hipStream_t s) {
    if (n <= 0) return MN_OK;
    if (n <= SC_TILE) {
        k_tile_scan<<<1, SC_THREADS, 0, s>>>(data, n, nullptr);
        MN_LAUNCH_CHECK("scan");
        return MN_OK;
    }
    int64_t nt = (n + SC_TILE - 1) / SC_TILE;
    k_tile_reduce<<<(unsigned)nt, SC_THREADS, 0, s>>>(data, n, partials);
    MN_LAUNCH_CHECK("scan reduce");
    int rc = scan_exclusive_u32(partials, nt, partials + nt, s);
    if (rc) return rc;
    k_tile_scan<<<(unsigned)nt, SC_THREADS, 0, s>>>(data, n, partials);
    MN_LAUNCH_CHECK("scan");
    return MN_OK;
}

int key_starts(const uint32_t *sorted_key, int64_t P, int64_t K, uint32_t kmask, int32_t *starts,
               hipStream_t s) {
    constexpr int per = KS_THREADS * KS_ITEMS;
    k_key_starts<<<(unsigned)((P + 1 + per - 1) / per), KS_THREADS, 0, s>>>(sorted_key, P, K,
                                                                            kmask, starts);
    MN_LAUNCH_CHECK("key starts");
    return MN_OK;
}

}  // namespace mn

using namespace mn;

namespace {

struct SortWs {
    uint32_t *kalt, *valt, *hist, *totals;
    uint32_t *calt[MN_SORT_MAX_COLS];
    int64_t bytes;
};

SortWs sort_layout(int64_t P, int ncols, char *base) {
    int64_t nblk = (P + RS_TILE - 1) / RS_TILE;
    int64_t nh = nblk * RS_RADIX;
    SortWs w{};
    int64_t off = 0;
    w.kalt = reinterpret_cast<uint32_t *>(base + off);
    off = align_up(off + 4 * P, 256);
    w.valt = reinterpret_cast<uint32_t *>(base + off);
    off = align_up(off + 4 * P, 256);
    for (int c = 0; c < ncols; ++c) {
        w.calt[c] = reinterpret_cast<uint32_t *>(base + off);
        off = align_up(off + 4 * P, 256);
    }
    w.hist = reinterpret_cast<uint32_t *>(base + off);
    off = align_up(off + 4 * nh, 256);
    w.totals = reinterpret_cast<uint32_t *>(base + off);
    off = align_up(off + 4 * RS_RADIX, 256);
    w.bytes = off;
    return w;
}

// ---- the no-allocation sort ----------------------------------------------
// Its workspace is this file-scope device array: each GPU the library runs on
// holds its own copy, at its own address, until the process ends. In host
// code the name `scratch` is only a stand-in for the symbol; the device
// address comes from hipGetSymbolAddress, taken once per device with that
// device current, and only that address is ever handed to a kernel.
constexpr int64_t kSortScratchBytes = int64_t(96) << 20;
static __device__ __align__(256) unsigned char scratch[kSortScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

int scratch_address(void **out) {
    int dev = -1;
    MN_HIP_CHECK(hipGetDevice(&dev));
    MN_REQUIRE(dev >= 0 && dev < kMaxDevices, "sort (no-alloc): device index out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        MN_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        MN_REQUIRE(p != nullptr, "sort (no-alloc): no device address for the scratch array");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return MN_OK;
}

}  // namespace

extern "C" {

int64_t mn_sort_workspace_bytes(int64_t P) { return mn_sort_pairs_workspace_bytes(P, 0); }

int64_t mn_sort_pairs_workspace_bytes(int64_t P, int ncols) {
    if (P < 1) P = 1;
    if (ncols < 0 || ncols > MN_SORT_MAX_COLS) return -1;
    return sort_layout(P, ncols, nullptr).bytes;
}

int mn_sort_pairs(int64_t P, int key_bits, const uint32_t *key_in, uint32_t *key_out,
                  uint32_t *perm_out, int ncols, const uint32_t *const *cols_in,
                  uint32_t *const *cols_out, void *ws, int64_t ws_bytes, mn_stream_t stream) {
    clear_error();
    MN_REQUIRE(P >= 1 && P < (int64_t(1) << 32), "sort: P must be in [1, 2^32)");
    MN_REQUIRE(key_bits >= 0 && key_bits <= 32, "sort: key_bits must be in [0, 32]");
    MN_REQUIRE(ncols >= 0 && ncols <= MN_SORT_MAX_COLS, "sort: ncols out of range");
    MN_REQUIRE(key_in && key_out && perm_out && ws, "sort: NULL pointer");
    MN_REQUIRE(key_in != key_out, "sort: key_in and key_out must differ");
    SortCols user{};
    for (int c = 0; c < ncols; ++c) {
        MN_REQUIRE(cols_in && cols_out && cols_in[c] && cols_out[c], "sort: NULL column");
        MN_REQUIRE(cols_in[c] != cols_out[c], "sort: column in and out must differ");
        user.in[c] = cols_in[c];
        user.out[c] = cols_out[c];
    }
    SortWs w = sort_layout(P, ncols, static_cast<char *>(ws));
    MN_REQUIRE(ws_bytes >= w.bytes, "sort: workspace too small");
    hipStream_t s = as_stream(stream);
    // Passes of at most 8 bits, the key split evenly over them (the first
    // ones a bit wider): a 22-bit key as 8 + 7 + 7 bits, so no pass has
    // 256 digits where 128 do
    const int npass = key_bits <= 0 ? 1 : (key_bits + 7) / 8;
    const uint32_t kmask = key_bits >= 32 ? 0xFFFFFFFFu : ((1u << key_bits) - 1u);
    const int64_t nblk = (P + RS_TILE - 1) / RS_TILE;
    const uint32_t *ksrc = key_in;
    const uint32_t *vsrc = nullptr;  // identity values on the first pass
    SortCols cur{};
    for (int c = 0; c < ncols; ++c) cur.in[c] = user.in[c];
    int shift = 0;
    for (int p = 0; p < npass; ++p) {
        const bool to_out = ((npass - 1 - p) % 2) == 0;
        uint32_t *kdst = to_out ? key_out : w.kalt;
        uint32_t *vdst = to_out ? perm_out : w.valt;
        for (int c = 0; c < ncols; ++c) cur.out[c] = to_out ? user.out[c] : w.calt[c];
        const int width = key_bits <= 0 ? 8 : key_bits / npass + (p < key_bits % npass ? 1 : 0);
        const uint32_t dmask = (1u << width) - 1u;
        k_radix_hist<<<(unsigned)nblk, RS_THREADS, 0, s>>>(ksrc, P, shift, kmask, dmask, w.hist,
                                                           nblk);
        MN_LAUNCH_CHECK("radix hist");
        k_digit_scan<<<dmask + 1, SC_THREADS, 0, s>>>(w.hist, nblk, w.totals);
        MN_LAUNCH_CHECK("radix digit scan");
        k_radix_scatter<<<(unsigned)nblk, ST_THREADS, 0, s>>>(ksrc, vsrc, P, shift, kmask, dmask,
                                                             w.hist, w.totals, nblk, kdst, vdst,
                                                             ncols, cur);
        MN_LAUNCH_CHECK("radix scatter");
        shift += width;
        ksrc = kdst;
        vsrc = vdst;
        for (int c = 0; c < ncols; ++c) cur.in[c] = cur.out[c];
    }
    return MN_OK;
}

int mn_sort_pairs_noalloc(int64_t P, int key_bits, const uint32_t *key_in, uint32_t *key_out,
                          uint32_t *perm_out, int ncols, const uint32_t *const *cols_in,
                          uint32_t *const *cols_out, mn_stream_t stream) {
    clear_error();
    MN_REQUIRE(P >= 1 && P < (int64_t(1) << 32), "sort: P must be in [1, 2^32)");
    MN_REQUIRE(ncols >= 0 && ncols <= MN_SORT_MAX_COLS, "sort: ncols out of range");
    const int64_t need = sort_layout(P, ncols, nullptr).bytes;
    if (need > kSortScratchBytes) {
        set_error("sort (no-alloc): P = " + std::to_string(P) + " with " + std::to_string(ncols) +
                  " payload columns needs " + std::to_string(need) +
                  " bytes of workspace, above the " + std::to_string(kSortScratchBytes) +
                  "-byte scratch array; use mn_sort_pairs with a workspace");
        return MN_EINVAL;
    }
    void *ws = nullptr;
    int rc = scratch_address(&ws);
    if (rc) return rc;
    return mn_sort_pairs(P, key_bits, key_in, key_out, perm_out, ncols, cols_in, cols_out, ws,
                         kSortScratchBytes, stream);
}

int mn_sort_keys(int64_t P, int key_bits, const uint32_t *key_in, uint32_t *key_out,
                 uint32_t *perm_out, void *ws, int64_t ws_bytes, mn_stream_t stream) {
    return mn_sort_pairs(P, key_bits, key_in, key_out, perm_out, 0, nullptr, nullptr, ws,
                         ws_bytes, stream);
}

int64_t mn_subproblem_workspace_bytes(const mn_bins *g) {
    if (check_bins(g)) return -1;
    int64_t nb = nbins_total(g);
    int64_t off = 0;
    off = align_up(off + 4 * nb, 256);        // bin start
    off = align_up(off + 4 * nb, 256);        // bin end
    off = align_up(off + 4 * (nb + 1), 256);  // subproblem offsets
    off = align_up(off + 4 * scan_partials_elems(nb + 1), 256);
    return off;
}

int mn_build_subproblems(const mn_bins *g, int64_t P, const uint32_t *sorted_key, int32_t msub,
                         int32_t *sub_info, int64_t max_sub, int64_t *nsub_out, void *ws,
                         int64_t ws_bytes, mn_stream_t stream) {
    clear_error();
    int rc = check_bins(g);
    if (rc) return rc;
    MN_REQUIRE(P >= 1 && P < (int64_t(1) << 31), "subproblems: P must be in [1, 2^31)");
    MN_REQUIRE(msub >= 1, "subproblems: msub must be >= 1");
    MN_REQUIRE(sorted_key && sub_info && nsub_out && ws, "subproblems: NULL pointer");
    int64_t need = mn_subproblem_workspace_bytes(g);
    MN_REQUIRE(ws_bytes >= need, "subproblems: workspace too small");
    int64_t nb = nbins_total(g);
    char *base = static_cast<char *>(ws);
    int64_t off = 0;
    int32_t *bstart = reinterpret_cast<int32_t *>(base + off);
    off = align_up(off + 4 * nb, 256);
    int32_t *bend = reinterpret_cast<int32_t *>(base + off);
    off = align_up(off + 4 * nb, 256);
    uint32_t *soff = reinterpret_cast<uint32_t *>(base + off);
    off = align_up(off + 4 * (nb + 1), 256);
    uint32_t *partials = reinterpret_cast<uint32_t *>(base + off);
    hipStream_t s = as_stream(stream);
    rc = fill_zero(bstart, 4 * nb, s);
    if (rc) return rc;
    rc = fill_zero(bend, 4 * nb, s);
    if (rc) return rc;
    k_bin_bounds<<<blocks_for(P, 256), 256, 0, s>>>(sorted_key, P, nb, bstart, bend);
    MN_LAUNCH_CHECK("bin bounds");
    k_bin_nsub<<<blocks_for(nb + 1, 256), 256, 0, s>>>(bstart, bend, nb, msub, soff);
    MN_LAUNCH_CHECK("bin nsub");
    rc = scan_exclusive_u32(soff, nb + 1, partials, s);
    if (rc) return rc;
    uint32_t total = 0;
    MN_HIP_CHECK(hipMemcpyAsync(&total, soff + nb, 4, hipMemcpyDeviceToHost, s));
    MN_HIP_CHECK(hipStreamSynchronize(s));
    if ((int64_t)total > max_sub) {
        set_error("subproblems: table capacity max_sub too small");
        return MN_EINVAL;
    }
    k_sub_fill<<<blocks_for(nb, 256), 256, 0, s>>>(bstart, bend, soff, nb, msub, sub_info);
    MN_LAUNCH_CHECK("subproblem fill");
    *nsub_out = (int64_t)total;
    return MN_OK;
}

int mn_bin_starts(const mn_bins *g, int64_t P, const uint32_t *sorted_key, int32_t *starts,
                  mn_stream_t stream) {
    clear_error();
    int rc = check_bins(g);
    if (rc) return rc;
    MN_REQUIRE(P >= 1 && P < (int64_t(1) << 31), "bin starts: P must be in [1, 2^31)");
    MN_REQUIRE(sorted_key && starts, "bin starts: NULL pointer");
    return key_starts(sorted_key, P, nbins_total(g), 0xFFFFFFFFu, starts, as_stream(stream));
}

}  // extern "C"
