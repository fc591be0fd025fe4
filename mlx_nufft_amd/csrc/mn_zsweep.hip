// Owner-computes 3D spread ("z-sweep"): no atomics, every fine-grid cell is
// written exactly once with a plain store.
//
// Layout. The grid is cut into 8x8 (x, y) column blocks; one wavefront owns
// a block over a z-segment (a multiple of 8 cells) and sweeps it upwards in
// z-chunks of 8 cells. The block's columns form four 4x4 "quadrants" by
// parity (x = 2i + qx, y = 2j + qy for i, j < 4), so that a lane's two x
// (and two y) columns are adjacent in memory; each quadrant keeps its
// z-window in two matrix-core accumulators (v_mfma_f32_16x16x32_f16 tiles:
// rows are the quadrant's 16 cells, columns 16 consecutive z-slots), one for
// the real and one for the imaginary part. The window spans the chunk being
// processed (slots 0..7) and the 8 cells above it, which the footprints of
// the chunk's points reach (w <= 8 taps from a first tap in the chunk).
//
// Point order. Points are sorted by a key that stops at the (block, chunk)
// of their first tap and below that groups them by class: for each axis, a
// reach code saying whether the footprint crosses into the next block and
// which halves of the two blocks it covers (zs_reach). With the class ranks
// of zs_rank, the points a block receives from itself and from its -x, -y
// and -xy neighbours in one chunk are four contiguous key ranges, found
// through zstart (first sorted index with a key at or above k). The sorted
// word carries the first tap's x, y cell in its block and its z cell in its
// chunk, so the sweep needs no cell indices.
//
// Per batch (up to 64 points of one chunk, a lane per point; the two-vector
// kernel takes 32-point batches with lane pairs, see its LP comment):
//  * the lane's W ES weights of each axis (3W evaluations) are computed in
//    the block of the previous batch's first K-step, where their VALU work
//    overlaps its MFMAs (measured 1.5-3 % faster than in the prologue);
//  * prologue: the lane writes the weights at their cells: x- and y-weights into the
//    point's row of the weight table (the block's 8 columns in order, zero
//    elsewhere; taps off the block land in unread padding), and B = c w_z,
//    already split into fp16 hi + lo, into four slot-major tables (re hi,
//    re lo, im hi, im lo; [slot][point], zero elsewhere).
//  * K-steps of 32 points: lane (li, lk) = (l % 16, l / 16) supplies
//    A[li][8 lk + t] and B[8 lk + t][li] for t < 8: it reads its 8 points'
//    weight pairs (columns 2 (li / 4) + {0, 1} and rows 2 (li % 4) + {0, 1},
//    one 8-byte read each) and its B column (one 16-byte read per table), and for
//    each quadrant forms A = wx wy and splits it -- hi = the f32 product
//    rounded toward zero to fp16 (a truncation, identical on every
//    conversion path), lo = fp16(fma(wx, wy, -hi)), which also keeps the f32
//    product's rounding, so hi + lo carries the exact product to about
//    2^-22 -- and accumulates hi*hi' + hi*lo' + lo*hi' into the quadrant's
//    real and imaginary tiles: 24 MFMAs per K-step, issued so that each
//    of the 8 tiles recurs only every 8th instruction. (Skipping quadrants
//    that none of a K-step's 32 points meets was measured: a K-step mixes
//    so many classes that it spared 3 % of the MFMAs and was no faster.)
// After a chunk, slots 0..7 are complete: lane (li < 8, lk) stores slot li
// of cells (2 lk + qx, 2 r + qy) straight from the accumulators (four lanes
// per column write one 64-byte run, aligned because segments and chunks
// start at multiples of 8 cells) with non-temporal stores, and DPP
// row_shl:8 shifts every accumulator down by 8 slots, filling zeros.
//
// Scale. A is stored times 2^14 (2^7 per axis) and B times 2^s, a per-wave
// power of two with |B| < 2^14: set by the first batch and lowered (the
// accumulators rescaled exactly) when a later batch brings a larger
// strength. Every scaling is an ldexp, so strengths anywhere in fp32's
// finite range keep fp16 operands in their normal range.
//
// Loads. Memory waits on this target count outstanding loads in issue order,
// and the compiler can only wait for "all but the newest n" when every load
// is certain to have been issued. So every lane issues a batch's loads
// outside any branch (idle lanes read element 0), the batch loop is unrolled
// three ways (a register copy of a value still loading would wait for it),
// and the range bounds of the next chunk are fetched while the current one
// is swept. The words, fractions and perm of batch k + 2 and the strengths
// of batch k + 1 are in flight while batch k is built and swept.
//
// ref: nd.py:492-579 (the reference's output-driven spread this replaces),
// nd.py:298-372 (its bin sort and subproblem tables).
#include <cstdlib>
#include <cstring>

#include "mn_common.h"
#include "mn_zsweep.h"

namespace mn {
namespace {

constexpr int ZB = kZsBlock;  // block size along x and y
constexpr int ZC = kZsChunk;  // z-steps per chunk
constexpr int NR = 4;         // key ranges per chunk: own, -x, -y, -xy
// Weight-table row (floats) for width W: the x-weight of block column X at
// XO + X and the y-weight of row Y at YO + Y, X, Y in [0, 8). A point writes
// its W taps at XO + ox + a (ox in [1 - W, 8)): the taps off the block land
// in the slots around the two data runs, which are never read, so a tap's
// slot is a constant offset from the point's base and needs no index
// arithmetic. XO and YO are even (8-byte pair reads); ROW is 2 mod 4, so the
// K-step's four lane groups, which read rows 8 apart, start 16 banks apart.
template <int W>
struct RowLayout {
    static constexpr int XO = (W - 1 + 1) & ~1;
    static constexpr int YO = (XO + W + 7 + 1) & ~1;
    static constexpr int ROW = ((YO + W + 7) + 3) / 4 * 4 + 2;
};
// (rows and B entries of the point positions just past a batch, 64..71 or
// 32..39, stay zero: K-step lanes past a batch part read this group)
// halves per B-table slot row of the one-vector kernel: 64 points + pad. 36 dwords: the 16 slots of a
// quarter-wave's 16-byte reads start 4 (9 li mod 16) banks in, all apart.
constexpr int BST = 72;
constexpr int kTab = 16 * BST;  // halves per B table

typedef float mf4 __attribute__((ext_vector_type(4)));
typedef float mf2 __attribute__((ext_vector_type(2)));
typedef _Float16 mh8 __attribute__((ext_vector_type(8)));

template <int SH>
__device__ __forceinline__ float row_shl_zero(float v) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 + SH, 0xf, 0xf, true));
}

// The four key ranges of a chunk: range r = source block (bit 0: the -x
// neighbour, bit 1: the -y neighbour) and the class ranks that reach this
// block from it.
struct Ranges {
    int bx, by, dbx, dby, nby, nzc, clast;
    const int32_t *zstart;
    // (st, en) of range `lane` (lanes 0..3) of chunk c (c = -1 is the last
    // chunk, periodically); an empty range (both zstart[0]) for other lanes
    // and for chunks past clast. The loaded values are returned as they are
    // (a select on them here would make the wave wait for every load in
    // flight, the prefetched point data included, as soon as they issue).
    __device__ __forceinline__ int2 fetch(int c, int lane) const {
        const int r = lane & 3;
        const bool ok = lane < NR && c <= clast;
        const int cc = c < 0 ? c + nzc : c;
        const int blk = (bx + (r & 1) * dbx) * nby + (by + ((r >> 1) & 1) * dby);
        const int lo = (r & 1) ? 3 : 0;
        const int hi = r == 0 ? 16 : (r == 1 ? 15 : 12);
        const int64_t kb = ok ? ((int64_t)blk * nzc + cc) * 16 : 0;
        return make_int2(zstart[kb + (ok ? lo : 0)], zstart[kb + (ok ? hi : 0)]);
    }
};

// The wave's position in the chunks of its segment (uniform): the current
// chunk c, its next batch element and element count, the range prefix
// bounds p1..p3 and offsets dj0..dj3 (sorted index = element + dj of its
// range), and the prefetched bounds of chunk pc. Chunks -1 and -2 are the
// last two of the grid, seen periodically below z = 0: chunk -1 starts the
// segment at z = 0 (window slot 0 at z = -8), and when n2 is not a multiple
// of 8 the last chunk holds fewer cells than can reach z = 0, so chunk -2 is
// swept first, at the same window position (see chunk_pos).
struct Cursor {
    int c, clast, bat, tot;
    int p1, p2, p3, dj0, dj1, dj2, dj3;
    int pc, nst, nen;
};

// Window chunk (slot 0 at z = 8 wc) and the offset added to a point's z cell
// in its chunk to give its slot, for chunk c: the identity for c >= 0; for
// the periodic chunks, z = 8 (c + nzc) + dz - n2 puts the first tap at slot
// dz + 8 nzc - n2 (chunk -1) or that minus 8 (chunk -2; a negative slot is a
// point that cannot reach z >= 0).
__device__ __forceinline__ void chunk_pos(int c, int wrap_off, int &wc, int &off) {
    wc = c < -1 ? -1 : c;
    off = c >= 0 ? 0 : (c == -1 ? wrap_off : wrap_off - ZC);
}

__device__ __forceinline__ void cur_fetch(Cursor &k, const Ranges &rg, int c, int lane) {
    const int2 b = rg.fetch(c, lane);
    k.pc = c;
    k.nst = b.x;
    k.nen = b.y;
}

// Make chunk c current and start fetching the bounds of chunk c + 1.
__device__ __forceinline__ void cur_load(Cursor &k, const Ranges &rg, int c, int lane) {
    if (k.pc != c) cur_fetch(k, rg, c, lane);
    const int st0 = __builtin_amdgcn_readlane(k.nst, 0), n0 = __builtin_amdgcn_readlane(k.nen, 0) - st0;
    const int st1 = __builtin_amdgcn_readlane(k.nst, 1), n1 = __builtin_amdgcn_readlane(k.nen, 1) - st1;
    const int st2 = __builtin_amdgcn_readlane(k.nst, 2), n2 = __builtin_amdgcn_readlane(k.nen, 2) - st2;
    const int st3 = __builtin_amdgcn_readlane(k.nst, 3), n3 = __builtin_amdgcn_readlane(k.nen, 3) - st3;
    k.c = c;
    k.bat = 0;
    k.p1 = n0;
    k.p2 = n0 + n1;
    k.p3 = n0 + n1 + n2;
    k.tot = k.p3 + n3;
    k.dj0 = st0;
    k.dj1 = st1 - k.p1;
    k.dj2 = st2 - k.p2;
    k.dj3 = st3 - k.p3;
    cur_fetch(k, rg, c + 1, lane);
}

// One lane's point of a batch, its loads issued (the strength, which needs
// src, is loaded one batch later). A batch takes up to NBP points (64, or 32
// when lanes l and l + 32 share a point) from the current chunk (part A,
// slots [0, nA)) and, when that chunk ends first, the head of the next chunk
// (part B, slots [oB, oB + nB) from the next multiple of 8), so that the
// prologue runs on full batches across chunk ends. With 32-point batches the
// lower lane of a pair loads the point's x fraction into fx, the upper its y
// fraction; fy is unused.
struct ZPoint {
    int cA, nA, cB, oB, nB;  // uniform; nA = 0: done
    bool valid, inB;
    int r;                   // the point's range (source block)
    uint32_t wd, src;        // sorted word; index of its strength in c
    float fx, fy, fz;
    float2 pv;               // prephase (1 if none)
};

template <bool PRE, int NBP>
__device__ __forceinline__ ZPoint zp_next(Cursor &k, const Ranges &rg, int lane,
                                          const uint32_t *__restrict__ perm,
                                          const uint32_t *__restrict__ word, const CF3s &frs,
                                          const float2 *__restrict__ pre) {
    // past exhausted (or empty) chunks: usually one step, straight-line code
    if (k.bat >= k.tot && k.c <= k.clast) {
        cur_load(k, rg, k.c + 1, lane);
        while (k.bat >= k.tot && k.c <= k.clast) cur_load(k, rg, k.c + 1, lane);
    }
    ZPoint q;
    const int lp = lane & (NBP - 1);  // the point's slot in the batch
    q.cA = k.c;
    q.nA = k.c <= k.clast ? min(NBP, k.tot - k.bat) : 0;
    q.cB = k.c + 1;
    q.oB = (q.nA + 7) & ~7;
    q.nB = 0;
    // part A: elements bat + lp of the current chunk
    const int eA = k.bat + lp;
    int r = (eA >= k.p1 ? 1 : 0) + (eA >= k.p2 ? 1 : 0) + (eA >= k.p3 ? 1 : 0);
    int dj = r == 0 ? k.dj0 : (r == 1 ? k.dj1 : (r == 2 ? k.dj2 : k.dj3));
    int e = eA;
    k.bat += q.nA;
    if (q.nA > 0 && q.oB < NBP && k.c + 1 <= k.clast) {
        // part B: the head of the next chunk, whose bounds were prefetched
        cur_load(k, rg, k.c + 1, lane);
        q.nB = min(NBP - q.oB, k.tot);
        k.bat = q.nB;
        if (lp >= q.oB) {
            e = lp - q.oB;
            r = (e >= k.p1 ? 1 : 0) + (e >= k.p2 ? 1 : 0) + (e >= k.p3 ? 1 : 0);
            dj = r == 0 ? k.dj0 : (r == 1 ? k.dj1 : (r == 2 ? k.dj2 : k.dj3));
        }
    }
    q.inB = lp >= q.oB;
    q.valid = lp < q.nA || (q.inB && lp < q.oB + q.nB);
    const uint32_t j = q.valid ? (uint32_t)(e + dj) : 0u;
    q.r = r;
    q.wd = word[j];
    if constexpr (NBP == 64) {
        q.fx = frs.p[0][j];
        q.fy = frs.p[1][j];
    } else {
        q.fx = frs.p[lane >> 5][j];
        q.fy = 0.f;
    }
    q.fz = frs.p[2][j];
    const uint32_t pj = (perm ? perm : word)[j];
    q.src = perm ? pj : j;
    if constexpr (PRE)
        q.pv = pre[j];
    else
        q.pv = make_float2(1.f, 0.f);
    return q;
}

// hi/lo fp16 halves of the products x[t] y[t] (t = 0..7): hi is the f32
// product rounded toward zero to fp16, lo = fp16(fma(x, y, -hi)), each lo
// one mixed-precision fma that reads hi as fp16 (v_fma_mix{lo,hi}_f16, two
// per pair, against a conversion, an fma and a conversion per value).
__device__ __forceinline__ void split_prod8(const float (&x)[8], const float (&y)[8], mh8 &hi,
                                            mh8 &lo) {
    typedef _Float16 mh2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int t = 0; t < 8; t += 2) {
        const auto h = __builtin_amdgcn_cvt_pkrtz(x[t] * y[t], x[t + 1] * y[t + 1]);
        hi[t] = h[0];
        hi[t + 1] = h[1];
        uint32_t hb, lb;
        __builtin_memcpy(&hb, &h, 4);
        asm("v_fma_mixlo_f16 %0, %1, %2, -%3 op_sel_hi:[0,0,1]\n\t"
            "v_fma_mixhi_f16 %0, %4, %5, -%3 op_sel:[0,0,1] op_sel_hi:[0,0,1]"
            : "=&v"(lb)
            : "v"(x[t]), "v"(y[t]), "v"(hb), "v"(x[t + 1]), "v"(y[t + 1]));
        mh2 l;
        __builtin_memcpy(&l, &lb, 4);
        lo[t] = l[0];
        lo[t + 1] = l[1];
    }
}

__device__ __forceinline__ int lane_id() { return (int)threadIdx.x; }

// Wave-wide maximum, over the lanes of mask m, of a small non-negative
// integer (< 512), by ballots.
__device__ __forceinline__ int masked_max9(int v, uint64_t m) {
    int r = 0;
#pragma unroll
    for (int b = 8; b >= 0; --b) {
        const int cand = r | (1 << b);
        if (__ballot(v >= cand) & m) r = cand;
    }
    return r;
}

#ifndef ZS_OCC
#define ZS_OCC 2
#endif
template <int W, bool PRE, int VB>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(ZS_OCC))) void
k_spread_zsweep(int n0, int n1, int n2, int nbx, int nby, int nzc, int zseg, int nseg,
                float bl2e, const int32_t *__restrict__ zstart, const uint32_t *__restrict__ perm,
                const uint32_t *__restrict__ word, CF3s frs, const float2 *__restrict__ c,
                int64_t cstride, const float2 *__restrict__ pre, float2 *__restrict__ grid,
                int64_t gstride) {
    static_assert(W >= 2 && W <= ZB && ZC + W - 1 <= 16, "footprint exceeds the 16 slots");
    static_assert(VB == 1 || VB == 2, "one or two strength vectors per wave");
    constexpr float kAxisScale = 128.0f;
    constexpr int XO = RowLayout<W>::XO, YO = RowLayout<W>::YO, ROW = RowLayout<W>::ROW;
    // Two vectors per wave take 32-point batches (LP: lanes l and l + 32
    // share a point): the lower lane evaluates its x weights and writes its
    // x row and vector 0's B column, the upper lane its y weights, y row and
    // vector 1's B column, and each evaluates half of its z weights (the
    // pair swaps them), so the prologue is one instruction stream for both
    // and the tables take 16 KB (two waves per SIMD; 64-point tables for two
    // vectors took 29 KB, 1.25 waves per SIMD).
    constexpr bool LP = VB == 2;
    constexpr int NBP = LP ? 32 : 64;          // points per batch
    constexpr int ZGP = NBP / 8;               // the always-zero group
    constexpr int BSTP = LP ? NBP + 8 : BST;   // halves per B-table slot row
    constexpr int kTabP = 16 * BSTP;           // halves per B table
    constexpr int HW = (W + 1) / 2;            // z weights per lane of a pair
    static_assert(!LP || BSTP % 4 == 0, "16-byte B reads");
    __shared__ __align__(16) float rows[(NBP + 8) * ROW];
    __shared__ __align__(16) _Float16 btab[VB][4 * kTabP];
    const bool lx = !LP || lane_id() < 32;  // x half of a lane pair (every lane when !LP)
    int bx, by, seg;
    zs_block(xcd_remap(blockIdx.x, (int64_t)nbx * nby * nseg), nbx, nby, bx, by, seg);
    // this wave's strength vectors and grids
    c += (int64_t)blockIdx.y * VB * cstride;
    grid += (int64_t)blockIdx.y * VB * gstride;
    const int z0 = seg * zseg, zend = min(z0 + zseg, n2);
    const int lane = threadIdx.x, li = lane & 15, lk = lane >> 4;
    const int bxm = bx == 0 ? nbx - 1 : bx - 1, bym = by == 0 ? nby - 1 : by - 1;
    // the periodic chunks below z = 0 sit this far up when n2 is not a
    // multiple of 8 (their first-tap cells end at n2, not at 8 nzc)
    const int wrap_off = ZC * nzc - n2;
    int sexp[VB];  // INT32_MIN: unset until the first batch
    mf4 are[VB][4], aim[VB][4];
#pragma unroll
    for (int v = 0; v < VB; ++v) {
        sexp[v] = INT32_MIN;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            are[v][q] = mf4{0.f, 0.f, 0.f, 0.f};
            aim[v][q] = mf4{0.f, 0.f, 0.f, 0.f};
        }
    }
    int zb = z0 - ZC;  // z of slot 0
    // cell (2 lk + qx, 2 r + qy) of the block at z: a wave-uniform column
    // base per (q, r) plus the lane's offset 2 lk n1 n2 + z (< 2^31: the key
    // space bounds n0 n1 n2 by 2^28)
    const int64_t gblk = ((int64_t)ZB * bx * n1 + ZB * by) * n2;
    const int loff = 2 * lk * n1 * n2;

    // Slots 0..7 are complete: store the owned ones, shift the window by 8.
    auto advance = [&]() __attribute__((always_inline)) {
        const int z = zb + li;
        if (li < ZC && z >= z0 && z < zend) {
#pragma unroll
            for (int v = 0; v < VB; ++v)
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float2 *gq = grid + v * gstride + gblk +
                                     ((int64_t)(q >> 1) * n1 + (q & 1) + 2 * r) * n2;
                        // streaming store: each cell is written once and
                        // next read by the FFT; kept out of the caches it
                        // leaves them to the point and strength reads
                        // (measured 0.1-0.16 ms less per 512^3 spread)
                        const mf2 val = {__builtin_amdgcn_ldexpf(are[v][q][r], -14 - sexp[v]),
                                         __builtin_amdgcn_ldexpf(aim[v][q][r], -14 - sexp[v])};
                        __builtin_nontemporal_store(val, reinterpret_cast<mf2 *>(gq + loff + z));
                    }
        }
#pragma unroll
        for (int v = 0; v < VB; ++v)
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    are[v][q][r] = row_shl_zero<ZC>(are[v][q][r]);
                    aim[v][q][r] = row_shl_zero<ZC>(aim[v][q][r]);
                }
        zb += ZC;
    };

    // the window moves up to chunk c (the cursor is chunk-major): usually
    // one step, straight-line code (a loop that stores makes the compiler
    // wait for every outstanding load before it)
    auto window_to = [&](int c) __attribute__((always_inline)) {
        const int zt = ZC * (c < -1 ? -1 : c);
        if (zb < zt) {
            advance();
            if (zb < zt) {
                advance();
                while (zb < zt) advance();
            }
        }
    };

    // the K-step of 32 points over the 8-point groups [gs, min(gs + 4, g1))
    // of the tables; lanes past g1 read the zero group
    auto kstep = [&](int gs, int g1) __attribute__((always_inline)) {
        const int pos = 8 * (gs + lk < g1 ? gs + lk : ZGP);
        float wx0[8], wx1[8], wy0[8], wy1[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float *rr = rows + (pos + t) * ROW;
            const float2 px = *reinterpret_cast<const float2 *>(rr + XO + 2 * (li >> 2));
            const float2 py = *reinterpret_cast<const float2 *>(rr + YO + 2 * (li & 3));
            wx0[t] = px.x;
            wx1[t] = px.y;
            wy0[t] = py.x;
            wy1[t] = py.y;
        }
        mh8 ah[4], al[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
            split_prod8((q >> 1) ? wx1 : wx0, (q & 1) ? wy1 : wy0, ah[q], al[q]);
        const int bo = li * BSTP + pos;
#pragma unroll
        for (int v = 0; v < VB; ++v) {
            const mh8 brh = *reinterpret_cast<const mh8 *>(&btab[v][bo]);
            const mh8 brl = *reinterpret_cast<const mh8 *>(&btab[v][kTabP + bo]);
            const mh8 bih = *reinterpret_cast<const mh8 *>(&btab[v][2 * kTabP + bo]);
            const mh8 bil = *reinterpret_cast<const mh8 *>(&btab[v][3 * kTabP + bo]);
            // consecutive MFMAs go to different accumulators: each of
            // the 8 tiles of a vector is used again only 8 instructions
            // later
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                are[v][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[q], brh, are[v][q], 0, 0, 0);
                aim[v][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[q], bih, aim[v][q], 0, 0, 0);
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                are[v][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[q], brl, are[v][q], 0, 0, 0);
                aim[v][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[q], bil, aim[v][q], 0, 0, 0);
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                are[v][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[q], brh, are[v][q], 0, 0, 0);
                aim[v][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[q], bih, aim[v][q], 0, 0, 0);
            }
        }
    };
    // K-steps of 32 points over the 8-point groups [g0, g1) (g0 < g1); extra()
    // runs in the block of the first one, whose MFMAs it can overlap
    auto ksteps = [&](int g0, int g1, auto extra) __attribute__((always_inline)) {
        kstep(g0, g1);
        extra();
        for (int gs = g0 + 4; gs < g1; gs += 4) kstep(gs, g1);
    };

    // the 3W ES weights of a point (x and y scaled by kAxisScale); the scaled
    // distance (a - f) 2/w of tap a is one fma. A lane pair (LP) splits them:
    // ew[0] holds the lane's x (lower lane) or y (upper lane) weights, ew[1]
    // z weights [0, HW) (lower) or [HW, 2 HW) (upper; tap W is a dummy when
    // W is odd).
    constexpr int NE = LP ? 2 : 3;
    auto es_eval = [&](const ZPoint &p, float (&ew)[NE][W]) __attribute__((always_inline)) {
        constexpr float ih = 2.0f / W;
        if constexpr (LP) {
            const float zo = lx ? 0.f : (float)HW * ih;
#pragma unroll
            for (int a = 0; a < W; ++a)
                ew[0][a] = zs_es(__builtin_fmaf(-p.fx, ih, (float)a * ih), bl2e) * kAxisScale;
#pragma unroll
            for (int a = 0; a < HW; ++a)
                ew[1][a] = zs_es(__builtin_fmaf(-p.fz, ih, zo + (float)a * ih), bl2e);
        } else {
#pragma unroll
            for (int a = 0; a < W; ++a) {
                const float ca = (float)a * ih;
                ew[0][a] = zs_es(__builtin_fmaf(-p.fx, ih, ca), bl2e) * kAxisScale;
                ew[1][a] = zs_es(__builtin_fmaf(-p.fy, ih, ca), bl2e) * kAxisScale;
                ew[2][a] = zs_es(__builtin_fmaf(-p.fz, ih, ca), bl2e);
            }
        }
    };
    constexpr int NV = LP ? 1 : VB;  // strength vectors a lane carries

    // batch p with its strengths cp and weights ew; computes ewn for the next
    // batch pn
    auto process = [&](const ZPoint &p, const float2 (&cp)[NV], const float (&ew)[NE][W],
                       const ZPoint &pn, float (&ewn)[NE][W]) __attribute__((always_inline)) {
        int wcA, offA, wcB, offB;
        chunk_pos(p.cA, wrap_off, wcA, offA);
        chunk_pos(p.cB, wrap_off, wcB, offB);
        const int off = p.inB ? offB : offA;
        // points of chunk -2 below the reach of z = 0 take no part
        const bool valid = p.valid && (int)(p.wd >> 29) + off >= 0;
        float2 cv[NV];
        if constexpr (LP) {
            // the lane's own vector (lower lanes 0, upper lanes 1); the scale
            // of vector v is checked over its half of the wave
            cv[0] = valid ? make_float2(cp[0].x * p.pv.x - cp[0].y * p.pv.y,
                                        cp[0].x * p.pv.y + cp[0].y * p.pv.x)
                          : make_float2(0.f, 0.f);
            const float mx = fmaxf(fabsf(cv[0].x), fabsf(cv[0].y));
            const int eb = (__float_as_int(mx) >> 23) & 0xff;
#pragma unroll
            for (int v = 0; v < VB; ++v) {
                const uint64_t hm = v ? 0xFFFFFFFF00000000ull : 0x00000000FFFFFFFFull;
                if (sexp[v] == INT32_MIN || (__ballot(eb > 140 - sexp[v]) & hm)) {
                    const int want = min(140 - masked_max9(eb, hm), 139);
                    if (sexp[v] != INT32_MIN) {
#pragma unroll
                        for (int q = 0; q < 4; ++q)
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                are[v][q][r] = __builtin_amdgcn_ldexpf(are[v][q][r], want - sexp[v]);
                                aim[v][q][r] = __builtin_amdgcn_ldexpf(aim[v][q][r], want - sexp[v]);
                            }
                    }
                    sexp[v] = want;
                }
            }
        }
#pragma unroll
        for (int v = 0; v < (LP ? 0 : VB); ++v) {
            cv[v] = valid ? make_float2(cp[v].x * p.pv.x - cp[v].y * p.pv.y,
                                        cp[v].x * p.pv.y + cp[v].y * p.pv.x)
                          : make_float2(0.f, 0.f);
            // the scale is lowered when a strength reaches 2^(141 - sexp - 127);
            // then the batch's largest strength is below 2^(e - 126)
            const float mx = fmaxf(fabsf(cv[v].x), fabsf(cv[v].y));
            const int eb = (__float_as_int(mx) >> 23) & 0xff;
            if (sexp[v] == INT32_MIN || __ballot(eb > 140 - sexp[v])) {
                const int want = min(140 - wave_max9(eb), 139);
                if (sexp[v] != INT32_MIN) {
#pragma unroll
                    for (int q = 0; q < 4; ++q)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            are[v][q][r] = __builtin_amdgcn_ldexpf(are[v][q][r], want - sexp[v]);
                            aim[v][q][r] = __builtin_amdgcn_ldexpf(aim[v][q][r], want - sexp[v]);
                        }
                }
                sexp[v] = want;  // below the old scale whenever one was set
            }
        }
        window_to(p.cA);
        __syncthreads();  // the previous batch's K-steps are done with the tables
        {
            if constexpr (LP) {
                float2 *rz = reinterpret_cast<float2 *>(rows + (lane & 31) * ROW + (lx ? XO : YO));
#pragma unroll
                for (int i = 0; i < 4; ++i) rz[i] = make_float2(0.f, 0.f);
            } else {
                float2 *rzx = reinterpret_cast<float2 *>(rows + lane * ROW + XO);
                float2 *rzy = reinterpret_cast<float2 *>(rows + lane * ROW + YO);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    rzx[i] = make_float2(0.f, 0.f);
                    rzy[i] = make_float2(0.f, 0.f);
                }
            }
            float4 *bz = reinterpret_cast<float4 *>(&btab[0][0]);
            constexpr int nb4 = VB * 4 * kTabP / 8;  // float4 count of the B tables
#pragma unroll
            for (int i = lane; i < nb4; i += 64) bz[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        __syncthreads();
        if constexpr (LP) {
            // the pair's z weights: each lane holds half and takes the other
            // half from its partner (every lane swaps, valid or not)
            float wz[W];
#pragma unroll
            for (int a = 0; a < HW; ++a) {
                const float mine = ew[1][a];
                const float oth = __shfl_xor(mine, 32, 64);
                wz[a] = lx ? mine : oth;
                if (HW + a < W) wz[HW + a] = lx ? oth : mine;
            }
            if (valid) {
                const int lp = lane & 31;
                const int ox = (int)((p.wd >> 23) & 7u) - ((p.r & 1) ? ZB : 0);
                const int oy = (int)((p.wd >> 26) & 7u) - ((p.r & 2) ? ZB : 0);
                const int sz = (int)(p.wd >> 29) + off;
                const int se = lx ? sexp[0] : sexp[1];
                const float2 cb = make_float2(__builtin_amdgcn_ldexpf(cv[0].x, se),
                                              __builtin_amdgcn_ldexpf(cv[0].y, se));
                float *rr = rows + lp * ROW + (lx ? XO + ox : YO + oy);
                _Float16 *bt = &btab[lx ? 0 : 1][0] + sz * BSTP + lp;
#pragma unroll
                for (int a = 0; a < W; ++a) {
                    rr[a] = ew[0][a];
                    _Float16 *o = bt + a * BSTP;
                    const auto h = __builtin_amdgcn_cvt_pkrtz(cb.x * wz[a], cb.y * wz[a]);
                    o[0] = h[0];
                    o[kTabP] = (_Float16)__builtin_fmaf(cb.x, wz[a], -(float)h[0]);
                    o[2 * kTabP] = h[1];
                    o[3 * kTabP] = (_Float16)__builtin_fmaf(cb.y, wz[a], -(float)h[1]);
                }
            }
        } else if (valid) {
            // first tap relative to this block (minus 8 for points of the -x
            // / -y neighbour blocks) and its slot in its chunk's window
            const int ox = (int)((p.wd >> 23) & 7u) - ((p.r & 1) ? ZB : 0);
            const int oy = (int)((p.wd >> 26) & 7u) - ((p.r & 2) ? ZB : 0);
            const int sz = (int)(p.wd >> 29) + off;
            float2 cb[VB];
#pragma unroll
            for (int v = 0; v < VB; ++v)
                cb[v] = make_float2(__builtin_amdgcn_ldexpf(cv[v].x, sexp[v]),
                                    __builtin_amdgcn_ldexpf(cv[v].y, sexp[v]));
            // tap a of each axis goes to a constant offset from the point's
            // base (taps off the block land in unread slots)
            float *rx = rows + lane * ROW + XO + ox;
            float *ry = rows + lane * ROW + YO + oy;
            _Float16 *bt = &btab[0][0] + sz * BST + lane;
#pragma unroll
            for (int a = 0; a < W; ++a) {
                rx[a] = ew[0][a];
                ry[a] = ew[1][a];
                const float wz = ew[2][a];
#pragma unroll
                for (int v = 0; v < VB; ++v) {
                    _Float16 *o = bt + v * 4 * kTab + a * BST;
                    const auto h = __builtin_amdgcn_cvt_pkrtz(cb[v].x * wz, cb[v].y * wz);
                    o[0] = h[0];
                    o[kTab] = (_Float16)__builtin_fmaf(cb[v].x, wz, -(float)h[0]);
                    o[2 * kTab] = h[1];
                    o[3 * kTab] = (_Float16)__builtin_fmaf(cb[v].y, wz, -(float)h[1]);
                }
            }
        }
        __syncthreads();
        // part A in its chunk's window, then part B in the next chunk's
        ksteps(0, (p.nA + 7) >> 3, [&]() __attribute__((always_inline)) { es_eval(pn, ewn); });
        if (p.nB > 0) {
            window_to(p.cB);
            ksteps(p.oB >> 3, (p.oB + p.nB + 7) >> 3, []() {});
        }
    };

    auto strengths = [&](const ZPoint &p, float2 (&cv)[NV]) __attribute__((always_inline)) {
        if constexpr (LP) {
            cv[0] = c[(lane >> 5) * cstride + p.src];
        } else {
#pragma unroll
            for (int v = 0; v < VB; ++v) cv[v] = c[v * cstride + p.src];
        }
    };

    // the zero group's rows (the B tables are cleared with every batch)
    for (int i = lane; i < 8 * ROW; i += 64) rows[8 * ZGP * ROW + i] = 0.f;
    const int clast = (zend - 1) / ZC;  // the last chunk of the segment
    const Ranges rg{bx, by, bxm - bx, bym - by, nby, nzc, clast, zstart};
    Cursor cur;
    cur.pc = INT32_MIN;
    cur.clast = clast;
    cur_load(cur, rg, (z0 == 0 && wrap_off > 0) ? -2 : z0 / ZC - 1, lane);
    ZPoint pa = zp_next<PRE, NBP>(cur, rg, lane, perm, word, frs, pre);
    float2 ca[NV], cb[NV], cc[NV];
    float ewa[NE][W], ewb[NE][W], ewc[NE][W];
    strengths(pa, ca);  // idle lanes read c[perm[0]]: their rows stay zero
    es_eval(pa, ewa);
    ZPoint pb = zp_next<PRE, NBP>(cur, rg, lane, perm, word, frs, pre);
    ZPoint pc;
    for (;;) {
        if (pa.nA == 0) break;
        pc = zp_next<PRE, NBP>(cur, rg, lane, perm, word, frs, pre);
        strengths(pb, cb);
        process(pa, ca, ewa, pb, ewb);
        if (pb.nA == 0) break;
        pa = zp_next<PRE, NBP>(cur, rg, lane, perm, word, frs, pre);
        strengths(pc, cc);
        process(pb, cb, ewb, pc, ewc);
        if (pc.nA == 0) break;
        pb = zp_next<PRE, NBP>(cur, rg, lane, perm, word, frs, pre);
        strengths(pa, ca);
        process(pc, cc, ewc, pa, ewa);
    }
#pragma unroll
    for (int v = 0; v < VB; ++v)
        if (sexp[v] == INT32_MIN) sexp[v] = 0;  // no points at all: the window holds zeros
    while (zb < zend) advance();
}

}  // namespace

int zsweep_check(const mn_bins *g) {
    MN_REQUIRE(g != nullptr && g->dim == 3, "zsweep: 3D geometry required");
    MN_REQUIRE(g->w >= 2 && g->w <= ZB, "zsweep: kernel width must be in [2, 8]");
    MN_REQUIRE(g->n[0] % ZB == 0 && g->n[1] % ZB == 0, "zsweep: n0, n1 must be multiples of 8");
    MN_REQUIRE(g->n[0] >= 2 * ZB && g->n[1] >= 2 * ZB, "zsweep: n0, n1 must be >= 16");
    MN_REQUIRE(g->n[2] >= ZC && g->n[2] < (int64_t(1) << 24), "zsweep: n2 must be in [8, 2^24)");
    MN_REQUIRE(zsweep_nkeys(g) <= (int64_t(1) << kZsKeyBits),
               "zsweep: key space above 2^23 (n0*n1*ceil(n2/8)/4)");
    return MN_OK;
}

int64_t zsweep_nkeys(const mn_bins *g) {
    return (g->n[0] / ZB) * (g->n[1] / ZB) * ((g->n[2] + ZC - 1) / ZC) * 16;
}

namespace {

bool zsweep_pairs() {
    const char *e = std::getenv("MN_ZSWEEP_PAIRS");
    return !(e && e[0] == '0' && e[1] == '\0');
}

struct ZArgs {
    const mn_bins *g;
    float beta;
    int zseg;
    const int32_t *zstart;
    const uint32_t *perm;
    const uint32_t *word;
    CF3s frs;
    const float2 *c, *pre;
    float2 *grid;
    int64_t B;  // strength vectors (c: B rows of P, grid: B grids)
    int64_t P;
    hipStream_t s;
};

template <int DIM, int W>
struct ZLaunch {
    static int run(const ZArgs &a) {
        if constexpr (DIM != 3 || W > ZB) {
            set_error("zsweep: unsupported dim/width");
            return MN_EINVAL;
        } else {
            const int n0 = (int)a.g->n[0], n1 = (int)a.g->n[1], n2 = (int)a.g->n[2];
            const int nbx = n0 / ZB, nby = n1 / ZB, nseg = (n2 + a.zseg - 1) / a.zseg;
            const int nzc = (n2 + ZC - 1) / ZC;
            const int64_t nw = (int64_t)nbx * nby * nseg;
            const float bl2e = (float)(a.beta * 1.4426950408889634);
            const int64_t gs = (int64_t)n0 * n1 * n2;
            // Batches of vectors: one wave per (block, pair of vectors), in
            // 32-point batches (the weights, point loads and A operands are
            // formed once for both vectors); an odd last vector, and single
            // vectors, take one wave per (block, vector). MN_ZSWEEP_PAIRS=0
            // in the environment gives every vector its own wave.
            int64_t B1 = a.B;
            if (a.B >= 2 && !a.pre && zsweep_pairs()) {
                const int64_t np = a.B / 2;
                k_spread_zsweep<W, false, 2><<<dim3((unsigned)nw, (unsigned)np), 64, 0, a.s>>>(
                    n0, n1, n2, nbx, nby, nzc, a.zseg, nseg, bl2e, a.zstart, a.perm, a.word,
                    a.frs, a.c, a.P, nullptr, a.grid, gs);
                MN_LAUNCH_CHECK("spread_zsweep (vector pairs)");
                if ((a.B & 1) == 0) return MN_OK;
                B1 = 1;
            }
            const float2 *c1 = a.c + (a.B - B1) * a.P;
            float2 *g1 = a.grid + (a.B - B1) * gs;
            const dim3 gridv((unsigned)nw, (unsigned)B1);
            if (a.pre)
                k_spread_zsweep<W, true, 1><<<gridv, 64, 0, a.s>>>(
                    n0, n1, n2, nbx, nby, nzc, a.zseg, nseg, bl2e, a.zstart, a.perm, a.word,
                    a.frs, c1, a.P, a.pre, g1, gs);
            else
                k_spread_zsweep<W, false, 1><<<gridv, 64, 0, a.s>>>(
                    n0, n1, n2, nbx, nby, nzc, a.zseg, nseg, bl2e, a.zstart, a.perm, a.word,
                    a.frs, c1, a.P, a.pre, g1, gs);
            MN_LAUNCH_CHECK("spread_zsweep");
            return MN_OK;
        }
    }
};

}  // namespace
}  // namespace mn

using namespace mn;

extern "C" {

int64_t mn_zsweep_nkeys(const mn_bins *g) {
    if (zsweep_check(g)) return -1;
    return zsweep_nkeys(g);
}

int mn_zsweep_starts(const mn_bins *g, int64_t P, const uint32_t *sorted_word, int32_t *zstart,
                     mn_stream_t stream) {
    clear_error();
    int rc = zsweep_check(g);
    if (rc) return rc;
    MN_REQUIRE(P >= 1 && P < (int64_t(1) << 31), "zsweep starts: P must be in [1, 2^31)");
    MN_REQUIRE(sorted_word && zstart, "zsweep starts: NULL pointer");
    return key_starts(sorted_word, P, zsweep_nkeys(g), kZsKeyMask, zstart, as_stream(stream));
}

static int zsweep_spread(const mn_bins *g, float beta, int64_t P, int64_t B, int zseg,
                         const int32_t *zstart, const uint32_t *perm, const uint32_t *sorted_word,
                         const float *const frs[3], const void *c, const void *pre, void *grid,
                         mn_stream_t stream) {
    clear_error();
    int rc = zsweep_check(g);
    if (rc) return rc;
    MN_REQUIRE(P >= 1 && P < (int64_t(1) << 31), "zsweep spread: P must be in [1, 2^31)");
    MN_REQUIRE(B >= 1 && B < 65536, "zsweep spread: B must be in [1, 65535]");
    MN_REQUIRE(zseg >= ZC && zseg % ZC == 0, "zsweep spread: zseg must be a positive multiple of 8");
    MN_REQUIRE(zstart && sorted_word && c && grid, "zsweep spread: NULL pointer");
    ZArgs a{};
    for (int d = 0; d < 3; ++d) {
        MN_REQUIRE(frs[d], "zsweep spread: NULL sorted fraction pointer");
        a.frs.p[d] = frs[d];
    }
    a.g = g;
    a.beta = beta;
    a.zseg = zseg;
    a.zstart = zstart;
    a.perm = perm;
    a.word = sorted_word;
    a.c = static_cast<const float2 *>(c);
    a.pre = static_cast<const float2 *>(pre);
    a.grid = static_cast<float2 *>(grid);
    a.B = B;
    a.P = P;
    a.s = as_stream(stream);
    return select_dim_w<ZLaunch>(3, g->w, a);
}

int mn_spread_zsweep(const mn_bins *g, float beta, int64_t P, int zseg, const int32_t *zstart,
                     const uint32_t *perm, const uint32_t *sorted_word,
                     const float *const frs[3], const void *c, const void *pre, void *grid,
                     mn_stream_t stream) {
    return zsweep_spread(g, beta, P, 1, zseg, zstart, perm, sorted_word, frs, c, pre, grid,
                         stream);
}

int mn_spread_zsweep_batch(const mn_bins *g, float beta, int64_t P, int64_t B, int zseg,
                           const int32_t *zstart, const uint32_t *perm,
                           const uint32_t *sorted_word, const float *const frs[3],
                           const void *cs, void *grids, mn_stream_t stream) {
    return zsweep_spread(g, beta, P, B, zseg, zstart, perm, sorted_word, frs, cs, nullptr, grids,
                         stream);
}

}  // extern "C"
