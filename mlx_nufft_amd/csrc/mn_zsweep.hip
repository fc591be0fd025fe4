// Owner-computes 3D spread ("z-sweep"): no atomics, every fine-grid cell is
// written exactly once with a plain store.
//
// Two kernels share the blocks, segments, point order and key ranges below:
// k_spread_zsweep_mfma (the default, described further down) keeps the
// z-window of each 4x4 column quadrant in a matrix-core accumulator, and
// k_spread_zsweep (MN_ZSWEEP_KERNEL=valu) keeps it in per-lane registers, as
// this first part describes.
//
// Layout. The grid is cut into 8x8 (x, y) column blocks. Each wavefront owns
// one block over a z-segment; each lane owns one column of the block (lanes
// grouped by 4x4 quadrant, below) and keeps a W-cell complex window
// [z, z + W) of its column in VGPRs. The
// wave sweeps z upwards: at each z it adds every point whose first tap is at
// z and whose footprint touches the block, then cell z is complete and is
// stored (staged in LDS so stores run along z), and the window shifts by one
// cell -- all register indices are compile-time constants.
//
// Point order. Points are sorted by key ((bx*nby + by)*n2 + z)*4 + classpos,
// where bx, by, z come from the first tap i1 and classpos encodes whether the
// footprint reaches the next block in x (cx) and in y (cy), ordered
// [00, 01, 11, 10]. Block b receives points from itself (all classes) and
// from its -x, -y and -xy neighbours with the reaching classes; with that
// order each of the four is one contiguous key range per z, located through
// zstart[key] (first sorted index with that key or above). The sorted word
// (zs_word) carries the first tap's cell inside its block above the key, so
// the sweep needs no cell indices.
//
// Per batch of up to 64 points (two z-steps), a lane-per-point prologue
// evaluates the ES weights once and writes a table row: the 8 x-weights of
// the block's columns times the strength (complex), the 8 y-weights and the
// W z-weights. Per z-step and 4x4 column quadrant, a list holds the byte
// offsets of the rows of the points that touch the quadrant; the 16 lanes
// of the quadrant walk it, each point costing 2 MULs and 2*W FMAs per lane.
// Loads are pipelined two batches deep: while batch k is built and swept,
// the strengths of batch k+1 and the words / fractions / perm of batch k+2
// are in flight.
//
// ref: nd.py:492-579 (the reference's output-driven spread this replaces),
// nd.py:298-372 (its bin sort and subproblem tables).
#include <cstdlib>
#include <cstring>

#include "mn_common.h"
#include "mn_cursor.h"

namespace mn {
namespace {

constexpr int ZB = kZsBlock;  // block size along x and y (lanes: 8 x 8)
constexpr int ZST = 4;     // z-slices staged in LDS per store
constexpr int ZCH = 2;     // z-steps per prologue batch
constexpr int UNR = 4;     // points per unrolled sweep step (then one at a time)
constexpr int NR = 4;      // key ranges per z: own, -x, -y, -xy
constexpr int REC = 36;    // floats per table row (32 used; the pad spreads rows over banks)

// Lane layout: the wave's 64 lanes form four 16-lane groups, one per 4x4
// quadrant of the 8x8 column block; lane l owns column
// (4*qx + ((l >> 2) & 3), 4*qy + (l & 3)) with (qx, qy) = (l >> 5, (l >> 4) & 1).
__device__ __forceinline__ int lane_cx(int l) { return ((l >> 5) << 2) + ((l >> 2) & 3); }
__device__ __forceinline__ int lane_cy(int l) { return (((l >> 4) & 1) << 2) + (l & 3); }

// Stage the finished cell of each column; every ZST z-slices (or at the
// segment end) the wave writes them out with ZST consecutive lanes per
// column storing ZST consecutive z.
__device__ __forceinline__ void store_stage(float2 (*stage)[64], float2 *__restrict__ grid,
                                            int lane, int s, int zw, int n1, int n2, int bx,
                                            int by, float wr, float wi, bool last) {
    static_assert(ZST == 2 || ZST == 4 || ZST == 8, "ZST lanes per column");
    stage[s][lane] = make_float2(wr, wi);
    if (s == ZST - 1 || last) {
        __syncthreads();
        const int zb = zw - s, nz = s + 1;
        for (int colb = 0; colb < 64; colb += 64 / ZST) {
            const int col = colb + lane / ZST, zo = lane % ZST;
            if (zo < nz) {
                const int gx = ZB * bx + lane_cx(col), gy = ZB * by + lane_cy(col);
                grid[((int64_t)gx * n1 + gy) * n2 + zb + zo] = stage[zo][col];
            }
        }
        __syncthreads();
    }
}

// One point of a quadrant list: the lane's column weight times the strength
// (vr, vi) and the point's z-weights, read from its table row at rec.
template <int W>
__device__ __forceinline__ void sweep_load(const char *rec, int xo, int yo, float &vr, float &vi,
                                           float (&wz)[ZB]) {
    const float2 wxc = *reinterpret_cast<const float2 *>(rec + xo);
    const float wyv = *reinterpret_cast<const float *>(rec + yo);
    const float4 z0 = *reinterpret_cast<const float4 *>(rec + 4 * 3 * ZB);
    wz[0] = z0.x, wz[1] = z0.y, wz[2] = z0.z, wz[3] = z0.w;
    if constexpr (W > 4) {
        const float4 z1 = *reinterpret_cast<const float4 *>(rec + 4 * (3 * ZB + 4));
        wz[4] = z1.x, wz[5] = z1.y, wz[6] = z1.z, wz[7] = z1.w;
    }
    vr = wxc.x * wyv;
    vi = wxc.y * wyv;
}

template <int W>
__device__ __forceinline__ void sweep_fma(float vr, float vi, const float (&wz)[ZB],
                                          float (&wre)[W], float (&wim)[W]) {
#pragma unroll
    for (int a = 0; a < W; ++a) {
        wre[a] = fmaf(vr, wz[a], wre[a]);
        wim[a] = fmaf(vi, wz[a], wim[a]);
    }
}

// The wave's position in the key ranges of one z-step pair (ZCH z-steps x
// NR source ranges): the pair's first z, the next batch element and the
// number of elements. All uniform across the wave.
struct ZCursor {
    int zc, bat, tot;
};

// The ranges of a group of ZC z-steps, in LDS (the wave reads them back
// with broadcast loads): element e of range q, with pf[q] <= e < pf[q + 1],
// is sorted point e + dj[q]; pf is the running sum of the range sizes.
template <int ZC>
struct __align__(16) ZRanges {
    static_assert(ZC >= 1 && ZC <= 8, "at most 32 ranges");
    int pf[ZC * NR];
    int dj[ZC * NR];
};

// The four source blocks of a block (itself, -x, -y, -xy) and the segment end.
struct ZBlocks {
    int bx, by, bxm, bym, nby;
    int n2, zend;
};

// Load the ranges of the group starting at zc: lane i < ZC * NR takes range
// q = i (z-step i / NR, source i % NR), then a shuffle scan forms pf.
template <int ZC>
__device__ __forceinline__ void zc_load(ZCursor &k, int zc, const ZBlocks b,
                                        const int32_t *__restrict__ zstart, ZRanges<ZC> &rg,
                                        int lane) {
    k.zc = zc;
    k.bat = 0;
    int st = 0, cnt = 0;
    if (lane < ZC * NR) {
        const int r = lane % NR, z = zc + lane / NR;
        if (z < b.zend) {
            const int zz = z < 0 ? z + b.n2 : z;
            // source r: bit 0 = -x neighbour, bit 1 = -y neighbour; its key
            // classes [lo, hi] are those that reach this block
            const int blk = ((r & 1) ? b.bxm : b.bx) * b.nby + ((r & 2) ? b.bym : b.by);
            const int lo = r == 0 ? 0 : (r == 2 ? 1 : 2), hi = (r & 2) ? 2 : 3;
            const int64_t kb = ((int64_t)blk * b.n2 + zz) * 4;
            st = zstart[kb + lo];
            cnt = zstart[kb + hi + 1] - st;
        }
    }
    int incl = cnt;
#pragma unroll
    for (int d = 1; d < ZC * NR; d <<= 1) {
        const int v = __shfl_up(incl, d, 64);
        incl += (lane >= d) ? v : 0;
    }
    if (lane < ZC * NR) {
        rg.pf[lane] = incl - cnt;
        rg.dj[lane] = st - (incl - cnt);
    }
    k.tot = __shfl(incl, ZC * NR - 1, 64);
}

// Advance past exhausted (or empty) groups; stops at the segment end.
template <int ZC>
__device__ __forceinline__ void zc_settle(ZCursor &k, const ZBlocks b,
                                          const int32_t *__restrict__ zstart, ZRanges<ZC> &rg,
                                          int lane) {
    while (k.bat >= k.tot && k.zc < b.zend) zc_load<ZC>(k, k.zc + ZC, b, zstart, rg, lane);
}

// One lane's point of a batch, its loads issued (the strength, which needs
// src, is loaded one batch later).
struct ZPoint {
    int zc, nb;          // the batch's pair and size (uniform; nb = 0: done)
    bool valid;
    int tsel, r;         // z-step within the group and source range
    uint32_t wd, src;    // sorted word; index of the strength in c
    float fx, fy, fz;
    float2 pv;           // prephase (1 if none)
};

template <int ZC>
__device__ __forceinline__ ZPoint zp_issue(ZCursor &k, const ZBlocks b, int lane,
                                           const int32_t *__restrict__ zstart, ZRanges<ZC> &rg,
                                           const uint32_t *__restrict__ perm,
                                           const uint32_t *__restrict__ word, const CF3s &frs,
                                           const float2 *__restrict__ pre) {
    ZPoint q;
    q.zc = k.zc;
    q.nb = k.zc < b.zend ? min(64, k.tot - k.bat) : 0;
    q.valid = lane < q.nb;
    q.tsel = -1;
    q.r = 0;
    q.wd = 0;
    q.src = 0;
    q.fx = q.fy = q.fz = 0.f;
    q.pv = make_float2(1.f, 0.f);
    if (q.valid) {
        // the element's range: the last q with pf[q] <= e (empty ranges
        // repeat pf and are passed over)
        int pf[ZC * NR], djs[ZC * NR];
#pragma unroll
        for (int s = 0; s < ZC * NR; s += 4) {
            const int4 pa = *reinterpret_cast<const int4 *>(rg.pf + s);
            const int4 da = *reinterpret_cast<const int4 *>(rg.dj + s);
            pf[s] = pa.x, pf[s + 1] = pa.y, pf[s + 2] = pa.z, pf[s + 3] = pa.w;
            djs[s] = da.x, djs[s + 1] = da.y, djs[s + 2] = da.z, djs[s + 3] = da.w;
        }
        const int e = k.bat + lane;
        int i = 0, dj = djs[0];
#pragma unroll
        for (int s = 1; s < ZC * NR; ++s) {
            const bool ge = e >= pf[s];
            i += ge ? 1 : 0;
            dj = ge ? djs[s] : dj;
        }
        q.tsel = i / NR;
        q.r = i % NR;
        const uint32_t j = (uint32_t)(e + dj);
        q.wd = word[j];
        q.fx = frs.p[0][j];
        q.fy = frs.p[1][j];
        q.fz = frs.p[2][j];
        q.src = perm ? perm[j] : j;
        if (pre) q.pv = pre[j];
    }
    if (k.zc < b.zend) {
        k.bat += 64;
        zc_settle<ZC>(k, b, zstart, rg, lane);
    }
    return q;
}

// The bounds of the MFMA kernel's key ranges (SweepCursor fetch): range
// i = (z-step i / NR, source i % NR) of the group starting at zc. Every lane
// loads (key 0 for lanes without a range), outside any branch.
struct ZFetch {
    int bx, by, dbx, dby, nby, n2, zend, nq;  // dbx = bxm - bx, dby = bym - by
    const int32_t *zstart;
    __device__ __forceinline__ int2 operator()(int zc, int lane) const {
        const int r = lane % NR, z = zc + lane / NR;
        const bool ok = lane < nq && z < zend;
        const int zz = z < 0 ? z + n2 : z;
        // source r: bit 0 = -x neighbour, bit 1 = -y neighbour (chosen by
        // arithmetic: a lane-dependent choice between two fields would put
        // the object in scratch); its key classes [lo, hi] are those that
        // reach this block
        const int blk = (bx + (r & 1) * dbx) * nby + (by + ((r >> 1) & 1) * dby);
        const int lo = r == 0 ? 0 : (r == 2 ? 1 : 2), hi = (r & 2) ? 2 : 3;
        const int64_t kb = ok ? ((int64_t)blk * n2 + zz) * 4 : 0;
        const int st = zstart[kb + (ok ? lo : 0)], en = zstart[kb + (ok ? hi + 1 : 0)];
        return make_int2(ok ? st : 0, ok ? en : 0);
    }
};

// The next batch of the MFMA kernel, its point loads issued by every lane
// (an idle lane reads element 0) outside any branch, so the compiler can
// wait for exactly the loads a later use needs.
template <int ZG, bool PRE>
__device__ __forceinline__ ZPoint zp_next(SweepCursor &k, const ZFetch zf, int lane,
                                          SweepRanges<ZG * NR> &rg, uint8_t *qidx,
                                          const uint32_t *__restrict__ perm,
                                          const uint32_t *__restrict__ word, const CF3s &frs,
                                          const float2 *__restrict__ pre) {
    const SweepBatch sb = sweep_next<ZG * NR, ZG>(k, zf.zend, rg, qidx, lane, zf);
    ZPoint q;
    q.zc = sb.zc;
    q.nb = sb.nb;
    q.valid = sb.valid;
    q.tsel = sb.valid ? sb.range / NR : -1;
    q.r = sb.range % NR;
    const uint32_t j = sb.j;
    q.wd = word[j];
    q.fx = frs.p[0][j];
    q.fy = frs.p[1][j];
    q.fz = frs.p[2][j];
    const uint32_t pj = (perm ? perm : word)[j];
    q.src = perm ? pj : j;
    if constexpr (PRE)
        q.pv = pre[j];
    else
        q.pv = make_float2(1.f, 0.f);
    return q;
}

// Workgroup index -> (column block bx, by; z-segment seg). The segment
// varies slowest; within a segment the blocks go in bands of ZS_BAND
// consecutive bx rows, bx fastest inside a band. The -x, -y and -xy
// neighbours of a block, which read the same reaching points, are then
// dispatched at most ZS_BAND + 1 workgroups earlier (except across a band
// edge) and run on the same XCD at about the same z. Measured on MI355X with
// 2e7 uniform points on a 512^3 grid: 18 % less HBM fetch than the
// segment-fastest order, and the same time within noise (the kernel is
// bound by instruction issue).
constexpr int ZS_BAND = 16;
__device__ __forceinline__ void zs_block(int64_t wid, int nbx, int nby, int &bx, int &by,
                                         int &seg) {
    const int64_t plane = (int64_t)nbx * nby;
    seg = (int)(wid / plane);
    const int64_t r = wid % plane, bandc = (int64_t)ZS_BAND * nby;
    const int b0 = (int)(r / bandc) * ZS_BAND;
    const int tx = min(ZS_BAND, nbx - b0);
    const int local = (int)(r % bandc);
    by = local / tx;
    bx = b0 + local % tx;
}

template <int W>
__global__ __launch_bounds__(64) void k_spread_zsweep(int n0, int n1, int n2, int nbx, int nby,
                                                      int zseg, int nseg, float bl2e,
                                                      float inv_hw,
                                                      const int32_t *__restrict__ zstart,
                                                      const uint32_t *__restrict__ perm,
                                                      const uint32_t *__restrict__ word,
                                                      CF3s frs,
                                                      const float2 *__restrict__ c,
                                                      const float2 *__restrict__ pre,
                                                      float2 *__restrict__ grid) {
    // table rows: x-weights of the block's 8 columns times the strength
    // (complex, 16 floats), y-weights of its 8 rows, W z-weights (padded to
    // 8); row 64 stays zero and pads the shorter quadrant lists, whose
    // entries are row byte offsets.
    __shared__ __align__(16) float table[(64 + 1) * REC];
    __shared__ __align__(16) uint16_t lists[ZCH][4][64];
    constexpr uint32_t kPad = 64u * REC * 4u;  // byte offset of the zero row
    __shared__ float2 stage[ZST][64];
    __shared__ ZRanges<ZCH> rg;
    int bx, by, seg;
    zs_block(xcd_remap(blockIdx.x, (int64_t)nbx * nby * nseg), nbx, nby, bx, by, seg);
    const int z0 = seg * zseg, zend = min(z0 + zseg, n2);
    const int lane = threadIdx.x, grp = lane >> 4;
    const int cxl = lane_cx(lane), cyl = lane_cy(lane);
    const int xo = 8 * cxl, yo = 4 * (2 * ZB + cyl);  // byte offsets of this lane's x / y weight
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    if (lane < REC) table[64 * REC + lane] = 0.f;
    ZBlocks bk;
    bk.bx = bx;
    bk.by = by;
    bk.bxm = bx == 0 ? nbx - 1 : bx - 1;
    bk.bym = by == 0 ? nby - 1 : by - 1;
    bk.nby = nby;
    bk.n2 = n2;
    bk.zend = zend;
    float wre[W], wim[W];
#pragma unroll
    for (int a = 0; a < W; ++a) wre[a] = wim[a] = 0.f;
    int zw = z0 - (W - 1);  // z of window cell 0

    // Software pipeline over batches: while batch p1 is built and swept,
    // the strengths of p2 and the words / fractions / perm of p3 load.
    ZCursor cur;
    zc_load<ZCH>(cur, z0 - (W - 1), bk, zstart, rg, lane);
    zc_settle<ZCH>(cur, bk, zstart, rg, lane);
    ZPoint p1 = zp_issue<ZCH>(cur, bk, lane, zstart, rg, perm, word, frs, pre);
    float2 c1 = p1.valid ? c[p1.src] : make_float2(0.f, 0.f);
    ZPoint p2 = zp_issue<ZCH>(cur, bk, lane, zstart, rg, perm, word, frs, pre);
    while (p1.nb > 0) {
        const float2 c2 = p2.valid ? c[p2.src] : make_float2(0.f, 0.f);
        const ZPoint p3 = zp_issue<ZCH>(cur, bk, lane, zstart, rg, perm, word, frs, pre);
        const int zc = p1.zc;
        __syncthreads();
#pragma unroll
        for (int k = 0; k < ZCH * 4 * 32; k += 64)
            reinterpret_cast<uint32_t *>(lists)[k + lane] = kPad | (kPad << 16);
        int touch = 0;
        if (p1.valid) {
            // first tap relative to this block: the word's in-block cell,
            // minus 8 for points of the -x / -y neighbour blocks
            const int ox = (int)((p1.wd >> kZsKeyBits) & 7u) - ((p1.r & 1) ? ZB : 0);
            const int oy = (int)((p1.wd >> (kZsKeyBits + 3)) & 7u) - ((p1.r & 2) ? ZB : 0);
            const float2 cv = make_float2(c1.x * p1.pv.x - c1.y * p1.pv.y,
                                          c1.x * p1.pv.y + c1.y * p1.pv.x);
            float4 *rec = reinterpret_cast<float4 *>(table + lane * REC);
            float wx[ZB], wy[ZB], wz[ZB];
            // scaled distance of column q from the point:
            // (q - (ox + fx)) * 2/W = q*2/W - (ox + fx)*2/W
            constexpr float ih = 2.0f / W;
            const float sx = ((float)ox + p1.fx) * ih, sy = ((float)oy + p1.fy) * ih;
            const float sz = p1.fz * ih;
#pragma unroll
            for (int q = 0; q < ZB; ++q) {
                const float ex = es_weight_z((float)q * ih - sx, bl2e);
                const float ey = es_weight_z((float)q * ih - sy, bl2e);
                wx[q] = ((unsigned)(q - ox) < (unsigned)W) ? ex : 0.f;
                wy[q] = ((unsigned)(q - oy) < (unsigned)W) ? ey : 0.f;
                wz[q] = q < W ? es_weight_z((float)q * ih - sz, bl2e) : 0.f;
            }
#pragma unroll
            for (int q = 0; q < ZB; q += 2)
                rec[q / 2] = make_float4(cv.x * wx[q], cv.y * wx[q], cv.x * wx[q + 1],
                                         cv.y * wx[q + 1]);
            rec[4] = make_float4(wy[0], wy[1], wy[2], wy[3]);
            rec[5] = make_float4(wy[4], wy[5], wy[6], wy[7]);
            rec[6] = make_float4(wz[0], wz[1], wz[2], wz[3]);
            rec[7] = make_float4(wz[4], wz[5], wz[6], wz[7]);
            // quadrants (qx, qy) the footprint [ox, ox + W) x [oy, oy + W) meets
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int qx = q >> 1, qy = q & 1;
                const bool hit = ox < 4 * qx + 4 && ox + W > 4 * qx && oy < 4 * qy + 4 &&
                                 oy + W > 4 * qy;
                touch |= hit ? (1 << q) : 0;
            }
        }
        // per z-step and quadrant: the batch rows that touch it, in order
        int cnt[ZCH][4];
#pragma unroll
        for (int t = 0; t < ZCH; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const bool mine = p1.tsel == t && ((touch >> q) & 1);
                const uint64_t bq = __ballot(mine);
                cnt[t][q] = __popcll(bq);
                if (mine) lists[t][q][__popcll(bq & lt_mask)] = (uint16_t)(lane * REC * 4);
            }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < ZCH; ++t) {
            const int nit = max(max(cnt[t][0], cnt[t][1]), max(cnt[t][2], cnt[t][3]));
            if (nit == 0) continue;
            const int ze = zc + t;
            while (zw < ze) {
                if (zw >= z0)
                    store_stage(stage, grid, lane, (zw - z0) % ZST, zw, n1, n2, bx, by,
                                wre[0], wim[0], zw == zend - 1);
#pragma unroll
                for (int a = 0; a < W - 1; ++a) {
                    wre[a] = wre[a + 1];
                    wim[a] = wim[a + 1];
                }
                wre[W - 1] = wim[W - 1] = 0.f;
                ++zw;
            }
            const uint16_t *lq = lists[t][grp];
            const char *tb = reinterpret_cast<const char *>(table);
            const int nit4 = nit & ~(UNR - 1);
            int it = 0;
            for (; it < nit4; it += UNR) {
                const uint2 pk = *reinterpret_cast<const uint2 *>(lq + it);
                const uint32_t off[UNR] = {pk.x & 0xffffu, pk.x >> 16, pk.y & 0xffffu,
                                           pk.y >> 16};
                float vr[UNR], vi[UNR], wzz[UNR][ZB];
#pragma unroll
                for (int u = 0; u < UNR; ++u)
                    sweep_load<W>(tb + off[u], xo, yo, vr[u], vi[u], wzz[u]);
#pragma unroll
                for (int u = 0; u < UNR; ++u) sweep_fma<W>(vr[u], vi[u], wzz[u], wre, wim);
            }
            for (; it < nit; ++it) {
                float vr, vi, wzz[ZB];
                sweep_load<W>(tb + lq[it], xo, yo, vr, vi, wzz);
                sweep_fma<W>(vr, vi, wzz, wre, wim);
            }
        }
        p1 = p2;
        c1 = c2;
        p2 = p3;
    }
    while (zw < zend) {  // drain the window up to the segment end
        if (zw >= z0)
            store_stage(stage, grid, lane, (zw - z0) % ZST, zw, n1, n2, bx, by, wre[0], wim[0],
                        zw == zend - 1);
#pragma unroll
        for (int a = 0; a < W - 1; ++a) {
            wre[a] = wre[a + 1];
            wim[a] = wim[a + 1];
        }
        wre[W - 1] = wim[W - 1] = 0.f;
        ++zw;
    }
}

// ---------------------------------------------------------------------------
// MFMA z-sweep: the same blocks, segments, point order and cursor as above,
// with the z-window held in matrix-core accumulators instead of per-lane
// registers.
//
// Each 4x4 column quadrant q = (qx, qy) of the block has one 16x16 f32
// accumulator: rows i are its cells (4qx + i/4, 4qy + i%4), columns
// j = 2s + ri are 8 z-slots (z = zb + s) times (re, im). A chunk is ZC
// consecutive z-steps [zb, zb + ZC) with ZC + W - 1 <= 8, so the footprint
// of every point whose first tap lies in the chunk fits the 8 slots. The
// cursor walks groups of G chunks and a batch holds up to 64 points of one
// group, in z-major order, so each chunk's points are consecutive lanes.
//
// A lane-per-point prologue writes each point's table row: the block's 8
// x-weights and 8 y-weights (zero outside the footprint), stored as pairs
// (w[a], w[a + 4]) so that one 8-byte read gives a lane its factor for both
// quadrant columns (rows), and B = strength x z-weight at the point's slot
// offset in its chunk (16 floats, j = 2s + ri). The sweep then takes the
// chunk's rows 4 at a time; per K-step every quadrant runs
// v_mfma_f32_16x16x4f32 with A[i][k] = wx[x_i] wy[y_i] (zero off the
// footprint) and the shared B[k][j]. Lane l supplies A[l % 16][l / 16] and
// B[l / 16][l % 16] and holds D[4 (l / 16) + r][l % 16] in element r. Every
// point costs 4 MFMAs / 4 and the lane 3 LDS reads and 4 MULs per K-step.
//
// For W <= ZM_F16_MAXW (6) the products run on the fp16 matrix path
// instead: K-steps of 16 points with v_mfma_f32_16x16x16f16, each f32
// operand split into fp16 hi + lo and the product taken as hi*hi' + hi*lo'
// + lo*hi' (about 2^-20 relative). On gfx950 f32 MFMAs and VALU
// instructions from waves sharing a SIMD do not overlap, but fp16 MFMAs
// mostly do, and they retire about 17x the MACs per cycle.
//
// When the sweep passes a chunk, its slots 0 .. ZC-1 are complete: they go
// to an LDS ring of RING z-cells per column (flushed as runs along z) and
// every accumulator register shifts down by ZC slots (2 ZC lanes) with one
// DPP row_shl, which fills the freed slots with zeros.
//
// Loads. Memory waits on this target count outstanding loads in issue order,
// and the compiler can only wait for "all but the newest n" when every load
// is certain to have been issued. So each batch's loads are issued by every
// lane outside any branch, the batch loop is unrolled three ways (a register
// copy of a value still loading would wait for it), and the key-range
// bounds of the next cursor group are fetched one group ahead. The words,
// fractions and perm of batch k + 2 and the strengths of batch k + 1 are in
// flight while batch k is built and swept.
#ifndef ZM_REC
#define ZM_REC 36
#endif
#ifndef ZM_UNR
#define ZM_UNR 2
#endif
constexpr int MREC = ZM_REC;  // floats per table row: wx pairs[8], wy pairs[8], B[16], pad
constexpr int RING = 8;       // z-cells per column in the store ring
constexpr int KUNR = ZM_UNR;  // K-steps per unrolled sweep iteration

template <int W>
constexpr int mfma_chunk() {
    return (9 - W) < 4 ? (9 - W) : 4;
}
// chunks per cursor group: groups of 6 - 8 z-steps (at most 32 key ranges)
template <int W>
constexpr int mfma_group() {
    return 8 / mfma_chunk<W>();
}

template <int SH>
__device__ __forceinline__ float row_shl_zero(float v) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 + SH, 0xf, 0xf, true));
}

// Write the ring's cells [fz, cz) of the owned segment (starting at z0) to
// the grid: 8 lanes per column, 8 columns per pass.
__device__ __forceinline__ void ring_flush(const float2 *ring, float2 *__restrict__ grid, int lane,
                                           int fz, int cz, int z0, int n1, int n2, int bx,
                                           int by) {
    __syncthreads();
    const int nz = cz - fz, zo = lane & 7;
#pragma unroll
    for (int pass = 0; pass < 8; ++pass) {
        const int col = pass * 8 + (lane >> 3);
        if (zo < nz) {
            const int gx = ZB * bx + (col >> 3), gy = ZB * by + (col & 7);
            grid[((int64_t)gx * n1 + gy) * n2 + fz + zo] =
                ring[col * RING + ((fz - z0 + zo) & (RING - 1))];
        }
    }
    __syncthreads();
}

typedef float mf4 __attribute__((ext_vector_type(4)));
typedef _Float16 mh4 __attribute__((ext_vector_type(4)));

// Widths up to ZM_F16_MAXW sweep with fp16 matrix products (below).
#ifndef ZM_F16_MAXW
#define ZM_F16_MAXW 6
#endif

// x = hi + lo with hi = x cut to fp16's 10 stored mantissa bits (exact in
// fp16 for |x| in its normal range, so every conversion path gives the same
// hi) and lo = fp16(x - hi), where x - hi is exact in fp32: about 21
// significant bits, so hi*hi' + hi*lo' + lo*hi' carries a product to about
// 2^-20. (Rounding hi instead lets the compiler derive the hi in lo and the hi
// fed to the MFMA by different roundings, which can differ by a whole ulp.)
__device__ __forceinline__ void split_f16(float x, _Float16 &hi, _Float16 &lo) {
    const float h = __int_as_float(__float_as_int(x) & 0xffffe000);
    hi = (_Float16)h;
    lo = (_Float16)(x - h);
}

#ifndef ZM_OCC
#define ZM_OCC 3
#endif
#define ZM_WPE __attribute__((amdgpu_waves_per_eu(ZM_OCC)))
template <int W, bool PRE>
__global__ __launch_bounds__(64) ZM_WPE void k_spread_zsweep_mfma(
    int n0, int n1, int n2, int nbx, int nby, int zseg, int nseg, float bl2e, float inv_hw,
    const int32_t *__restrict__ zstart, const uint32_t *__restrict__ perm,
    const uint32_t *__restrict__ word, CF3s frs, const float2 *__restrict__ c,
    const float2 *__restrict__ pre, float2 *__restrict__ grid) {
    constexpr int ZC = mfma_chunk<W>(), G = mfma_group<W>(), ZG = ZC * G;
    static_assert(ZC + W - 1 <= 8 && ZC <= RING, "chunk footprint exceeds the 8 slots");
    // fp16 products: A = wx wy is stored scaled by 2^14 (2^7 per axis) and
    // B = strength x wz by 2^sexp, a power of two per wave chosen so that
    // |B| < 2^14, which keeps both inside fp16's normal range; the
    // accumulators hold the grid times 2^(14 + sexp) and cells are scaled
    // back when they leave the window.
    constexpr bool F16 = W <= ZM_F16_MAXW;
    constexpr float kAxisScale = F16 ? 128.0f : 1.0f;
    int sexp = INT32_MIN;  // unset until the first batch with a nonzero strength
    float unscale = 1.0f;  // 2^-(14 + sexp)
    float bscale = 1.0f;   // 2^sexp
    __shared__ __align__(16) float table[(64 + 1) * MREC];
    __shared__ __align__(16) float2 ring[64 * RING];
    __shared__ SweepRanges<ZG * NR> rg;
    __shared__ uint8_t qidx[64];
    constexpr uint32_t kPad = 64u * MREC * 4u;  // byte offset of the zero row
    int bx, by, seg;
    zs_block(xcd_remap(blockIdx.x, (int64_t)nbx * nby * nseg), nbx, nby, bx, by, seg);
    const int z0 = seg * zseg, zend = min(z0 + zseg, n2);
    const int lane = threadIdx.x, li = lane & 15, lk = lane >> 4;
    if (lane < MREC) table[64 * MREC + lane] = 0.f;
    // byte offsets, within a table row, of this lane's wx pair, wy pair and B
    const int xo = 8 * (li >> 2), yo = 4 * ZB + 8 * (li & 3), bo = 4 * 2 * ZB + 4 * li;
    ZBlocks bk;
    bk.bx = bx;
    bk.by = by;
    bk.bxm = bx == 0 ? nbx - 1 : bx - 1;
    bk.bym = by == 0 ? nby - 1 : by - 1;
    bk.nby = nby;
    bk.n2 = n2;
    bk.zend = zend;
    mf4 acc[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[q] = mf4{0.f, 0.f, 0.f, 0.f};
    int zb = z0 - (W - 1);  // z of slot 0
    int fz = z0, cz = z0;   // owned cells [z0, fz) are stored, [fz, cz) sit in the ring

    // Slots 0 .. ZC-1 are complete: stage the owned ones in the ring, then
    // shift every accumulator down by ZC slots.
    // Cells leave the ring in whole groups of 4 z-cells from z0 (32-byte
    // aligned runs of a column when z0 is a multiple of 4), so no sector is
    // written twice; at most 3 cells wait, and with ZC <= 4 new ones the
    // ring never holds more than 7.
    static_assert(RING >= 3 + ZC, "store ring too small");
    auto advance = [&]() {
        const int lo = max(zb, z0), hi = min(zb + ZC, zend);
        if (lo < hi) {
            const int s = li >> 1, z = zb + s;
            if (s < ZC && z >= lo && z < hi) {
                float *rf = reinterpret_cast<float *>(ring) + ((z - z0) & (RING - 1)) * 2 + (li & 1);
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int col = (4 * (q >> 1) + lk) * ZB + 4 * (q & 1) + r;
                        rf[col * RING * 2] = acc[q][r] * unscale;
                    }
            }
            cz = hi;
            const int f4 = z0 + ((cz - z0) & ~3);
            if (f4 > fz) {
                ring_flush(ring, grid, lane, fz, f4, z0, n1, n2, bx, by);
                fz = f4;
            }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[q][r] = row_shl_zero<2 * ZC>(acc[q][r]);
        zb += ZC;
    };

    // Build and sweep one batch p whose strengths are cp.
    auto process = [&](const ZPoint &p, const float2 cp) __attribute__((always_inline)) {
        const int pch = p.tsel / ZC;  // the point's chunk in the group
        __syncthreads();
        const float2 cv = p.valid ? make_float2(cp.x * p.pv.x - cp.y * p.pv.y,
                                                cp.x * p.pv.y + cp.y * p.pv.x)
                                  : make_float2(0.f, 0.f);
        if constexpr (F16) {
            // the batch's largest strength is below 2^e
            const float mx = fmaxf(fabsf(cv.x), fabsf(cv.y));
            int e = ((__float_as_int(mx) >> 23) & 0xff) - 126;
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) e = max(e, __shfl_xor(e, off, 64));
            const int want = min(max(14 - e, -100), 100);
            if (sexp == INT32_MIN || want < sexp) {
                if (sexp != INT32_MIN) {
                    // a larger strength than before: rescale what is held
                    const float f = __builtin_amdgcn_ldexpf(1.0f, want - sexp);
#pragma unroll
                    for (int q = 0; q < 4; ++q)
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[q][r] *= f;
                }
                sexp = want;
                bscale = __builtin_amdgcn_ldexpf(1.0f, sexp);
                unscale = __builtin_amdgcn_ldexpf(1.0f, -14 - sexp);
            }
        }
        if (p.valid) {
            // first tap relative to this block (minus 8 for points of the -x
            // / -y neighbour blocks) and its slot in the chunk
            const int ox = (int)((p.wd >> kZsKeyBits) & 7u) - ((p.r & 1) ? ZB : 0);
            const int oy = (int)((p.wd >> (kZsKeyBits + 3)) & 7u) - ((p.r & 2) ? ZB : 0);
            const int dz = p.tsel - pch * ZC;
            static_assert(MREC % 2 == 0, "table rows hold float2 pairs");
            constexpr float ih = 2.0f / W;
            const float sx = ((float)ox + p.fx) * ih, sy = ((float)oy + p.fy) * ih;
            const float sz = p.fz * ih;
            float wx[ZB], wy[ZB], bz[ZB];
#pragma unroll
            for (int q = 0; q < ZB; ++q) {
                const float ex = es_weight_z((float)q * ih - sx, bl2e);
                const float ey = es_weight_z((float)q * ih - sy, bl2e);
                const float ez = es_weight_z((float)(q - dz) * ih - sz, bl2e);
                wx[q] = ((unsigned)(q - ox) < (unsigned)W) ? ex : 0.f;
                wy[q] = ((unsigned)(q - oy) < (unsigned)W) ? ey : 0.f;
                bz[q] = ((unsigned)(q - dz) < (unsigned)W) ? ez : 0.f;
            }
            // row: wx pairs (wx[a], wx[a + 4]), wy pairs, then B[2s + ri]
            float2 *rec2 = reinterpret_cast<float2 *>(table + lane * MREC);
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                rec2[a] = make_float2(wx[a] * kAxisScale, wx[a + 4] * kAxisScale);
                rec2[4 + a] = make_float2(wy[a] * kAxisScale, wy[a + 4] * kAxisScale);
            }
            const float2 cb = make_float2(cv.x * bscale, cv.y * bscale);
#pragma unroll
            for (int q = 0; q < ZB; ++q) rec2[8 + q] = make_float2(cb.x * bz[q], cb.y * bz[q]);
        }
        // each chunk's points: lanes [lo, lo + n) of the batch
        int nn[G], lo[G];
#pragma unroll
        for (int ch = 0; ch < G; ++ch) {
            nn[ch] = __popcll(__ballot(p.valid && pch == ch));
            lo[ch] = ch == 0 ? 0 : lo[ch - 1] + nn[ch - 1];
        }
        __syncthreads();
        const char *tb = reinterpret_cast<const char *>(table);
#pragma unroll
        for (int ch = 0; ch < G; ++ch) {
            // a chunk with points in this batch: every earlier chunk is
            // complete (the cursor is z-major), so the window moves up to it
            const int n = nn[ch];
            if (n == 0) continue;
            // usually one chunk: the first two steps are straight-line code,
            // so only a longer jump enters a loop (a loop that stores makes the
            // compiler wait for every outstanding load before it)
            const int zt = p.zc + ch * ZC;
            if (zb < zt) {
                advance();
                if (zb < zt) {
                    advance();
                    while (zb < zt) advance();
                }
            }
            if constexpr (F16) {
                // K-steps of 16 points: lane group lk supplies points
                // 4 lk .. 4 lk + 3 of the step (A[i][k], B[k][j] for
                // k = 4 lk + t), each product as hi*hi + hi*lo + lo*hi
                for (int e0 = 0; e0 < n; e0 += 16) {
                    mh4 ah[4], al[4], bh, bl;
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const int e = e0 + 4 * lk + t;
                        const uint32_t rb = e < n ? (uint32_t)(lo[ch] + e) * (MREC * 4u) : kPad;
                        const float2 px = *reinterpret_cast<const float2 *>(tb + rb + xo);
                        const float2 py = *reinterpret_cast<const float2 *>(tb + rb + yo);
                        const float bv = *reinterpret_cast<const float *>(tb + rb + bo);
                        const float a4[4] = {px.x * py.x, px.x * py.y, px.y * py.x, px.y * py.y};
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            _Float16 h, l;
                            split_f16(a4[q], h, l);
                            ah[q][t] = h;
                            al[q][t] = l;
                        }
                        _Float16 h, l;
                        split_f16(bv, h, l);
                        bh[t] = h;
                        bl[t] = l;
                    }
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        acc[q] = __builtin_amdgcn_mfma_f32_16x16x16f16(ah[q], bh, acc[q], 0, 0, 0);
                        acc[q] = __builtin_amdgcn_mfma_f32_16x16x16f16(ah[q], bl, acc[q], 0, 0, 0);
                        acc[q] = __builtin_amdgcn_mfma_f32_16x16x16f16(al[q], bh, acc[q], 0, 0, 0);
                    }
                }
            } else {
                for (int e0 = 0; e0 < n; e0 += 4 * KUNR) {
                    float av[KUNR][4], bv[KUNR];
    #pragma unroll
                    for (int u = 0; u < KUNR; ++u) {
                        const int e = e0 + 4 * u + lk;
                        const uint32_t rb = e < n ? (uint32_t)(lo[ch] + e) * (MREC * 4u) : kPad;
                        const float2 px = *reinterpret_cast<const float2 *>(tb + rb + xo);
                        const float2 py = *reinterpret_cast<const float2 *>(tb + rb + yo);
                        bv[u] = *reinterpret_cast<const float *>(tb + rb + bo);
                        av[u][0] = px.x * py.x;  // q = 0: (qx, qy) = (0, 0)
                        av[u][1] = px.x * py.y;  // q = 1: (0, 1)
                        av[u][2] = px.y * py.x;  // q = 2: (1, 0)
                        av[u][3] = px.y * py.y;  // q = 3: (1, 1)
                    }
    #pragma unroll
                    for (int u = 0; u < KUNR; ++u)
    #pragma unroll
                        for (int q = 0; q < 4; ++q)
                            acc[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u][q], bv[u], acc[q],
                                                                          0, 0, 0);
                }
            }
        }
    };

    // The batch loop, unrolled three ways with rotating names (A, B, C) so
    // that no register still being loaded is copied (a copy would wait for
    // it): each stage issues the loads of the batch two ahead, gathers the
    // strengths of the next one, then builds and sweeps the current one.
    const ZFetch zf{bk.bx, bk.by, bk.bxm - bk.bx, bk.bym - bk.by, nby, n2, zend, ZG * NR, zstart};
    SweepCursor cur;
    cur.pzc = INT32_MIN;
    sweep_load<ZG * NR, ZG>(cur, z0 - (W - 1), rg, lane, zf);
    ZPoint pa = zp_next<ZG, PRE>(cur, zf, lane, rg, qidx, perm, word, frs, pre);
    float2 ca = c[pa.src];  // idle lanes read c[perm[0]]: their rows are never used
    ZPoint pb = zp_next<ZG, PRE>(cur, zf, lane, rg, qidx, perm, word, frs, pre);
    ZPoint pc;
    float2 cb, cc;
    for (;;) {
        if (pa.nb == 0) break;
        pc = zp_next<ZG, PRE>(cur, zf, lane, rg, qidx, perm, word, frs, pre);
        cb = c[pb.src];
        process(pa, ca);
        if (pb.nb == 0) break;
        pa = zp_next<ZG, PRE>(cur, zf, lane, rg, qidx, perm, word, frs, pre);
        cc = c[pc.src];
        process(pb, cb);
        if (pc.nb == 0) break;
        pb = zp_next<ZG, PRE>(cur, zf, lane, rg, qidx, perm, word, frs, pre);
        ca = c[pa.src];
        process(pc, cc);
    }
    while (zb < zend) advance();
    if (cz > fz) ring_flush(ring, grid, lane, fz, cz, z0, n1, n2, bx, by);
}

}  // namespace

int zsweep_check(const mn_bins *g) {
    MN_REQUIRE(g != nullptr && g->dim == 3, "zsweep: 3D geometry required");
    MN_REQUIRE(g->w >= 2 && g->w <= ZB, "zsweep: kernel width must be in [2, 8]");
    MN_REQUIRE(g->n[0] % ZB == 0 && g->n[1] % ZB == 0, "zsweep: n0, n1 must be multiples of 8");
    MN_REQUIRE(g->n[0] >= 2 * ZB && g->n[1] >= 2 * ZB, "zsweep: n0, n1 must be >= 16");
    MN_REQUIRE(g->n[2] >= g->w && g->n[2] < (int64_t(1) << 24), "zsweep: n2 out of range");
    MN_REQUIRE(zsweep_nkeys(g) <= (int64_t(1) << kZsKeyBits),
               "zsweep: key space above 2^26 (n0*n1*n2/16)");
    return MN_OK;
}

int64_t zsweep_nkeys(const mn_bins *g) {
    return (g->n[0] / ZB) * (g->n[1] / ZB) * g->n[2] * 4;
}

namespace {

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
    hipStream_t s;
    bool valu;  // per-lane register windows instead of MFMA accumulators
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
            const int64_t nw = (int64_t)nbx * nby * nseg;
            const float bl2e = (float)(a.beta * 1.4426950408889634);
            const float inv_hw = (float)(2.0 / W);
            if (a.valu)
                k_spread_zsweep<W><<<(unsigned)nw, 64, 0, a.s>>>(
                    n0, n1, n2, nbx, nby, a.zseg, nseg, bl2e, inv_hw, a.zstart, a.perm, a.word,
                    a.frs, a.c, a.pre, a.grid);
            else if (a.pre)
                k_spread_zsweep_mfma<W, true><<<(unsigned)nw, 64, 0, a.s>>>(
                    n0, n1, n2, nbx, nby, a.zseg, nseg, bl2e, inv_hw, a.zstart, a.perm, a.word,
                    a.frs, a.c, a.pre, a.grid);
            else
                k_spread_zsweep_mfma<W, false><<<(unsigned)nw, 64, 0, a.s>>>(
                    n0, n1, n2, nbx, nby, a.zseg, nseg, bl2e, inv_hw, a.zstart, a.perm, a.word,
                    a.frs, a.c, a.pre, a.grid);
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

int mn_spread_zsweep(const mn_bins *g, float beta, int64_t P, int zseg, const int32_t *zstart,
                     const uint32_t *perm, const uint32_t *sorted_word,
                     const float *const frs[3], const void *c, const void *pre, void *grid,
                     mn_stream_t stream) {
    clear_error();
    int rc = zsweep_check(g);
    if (rc) return rc;
    MN_REQUIRE(P >= 1 && P < (int64_t(1) << 31), "zsweep spread: P must be in [1, 2^31)");
    MN_REQUIRE(zseg >= 1, "zsweep spread: zseg must be >= 1");
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
    a.s = as_stream(stream);
    const char *kv = getenv("MN_ZSWEEP_KERNEL");
    a.valu = kv && strcmp(kv, "valu") == 0;
    return select_dim_w<ZLaunch>(3, g->w, a);
}

}  // extern "C"
