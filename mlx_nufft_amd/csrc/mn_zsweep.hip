// Owner-computes 3D spread ("z-sweep"): no atomics, every fine-grid cell is
// written exactly once with a plain store.
//
// Layout. The grid is cut into 8x8 (x, y) column blocks. Each wavefront owns
// one block over a z-segment; lane (lx, ly) owns column (8 bx + lx, 8 by + ly)
// and keeps a W-cell complex window [z, z + W) of its column in VGPRs. The
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
// W z-weights. The sweep then costs each point 2*W FMAs per lane.
//
// ref: nd.py:492-579 (the reference's output-driven spread this replaces),
// nd.py:298-372 (its bin sort and subproblem tables).
#include "mn_common.h"

namespace mn {
namespace {

constexpr int ZB = kZsBlock;  // block size along x and y (lanes: 8 x 8)
constexpr int ZST = 4;     // z-slices staged in LDS per store
constexpr int ZCH = 2;     // z-steps per prologue batch
constexpr int UNR = 4;     // points per unrolled sweep step
constexpr int NR = 4;      // key ranges per z: own, -x, -y, -xy
constexpr int REC = 32;    // floats per table row

// Lane layout: the wave's 64 lanes form four 16-lane groups, one per 4x4
// quadrant of the 8x8 column block; lane l owns column
// (4*qx + ((l >> 2) & 3), 4*qy + (l & 3)) with (qx, qy) = (l >> 5, (l >> 4) & 1).
__device__ __forceinline__ int lane_cx(int l) { return ((l >> 5) << 2) + ((l >> 2) & 3); }
__device__ __forceinline__ int lane_cy(int l) { return (((l >> 4) & 1) << 2) + (l & 3); }

// Stage the finished cell of each column; every ZST z-slices (or at the
// segment end) the wave writes them out with 4 consecutive lanes per column
// storing 4 consecutive z.
__device__ __forceinline__ void store_stage(float2 (*stage)[64], float2 *__restrict__ grid,
                                            int lane, int s, int zw, int n1, int n2, int bx,
                                            int by, float wr, float wi, bool last) {
    stage[s][lane] = make_float2(wr, wi);
    if (s == ZST - 1 || last) {
        __syncthreads();
        const int zb = zw - s, nz = s + 1;
        for (int colb = 0; colb < 64; colb += 16) {
            const int col = colb + (lane >> 2), zo = lane & 3;
            if (zo < nz) {
                const int gx = ZB * bx + lane_cx(col), gy = ZB * by + lane_cy(col);
                grid[((int64_t)gx * n1 + gy) * n2 + zb + zo] = stage[zo][col];
            }
        }
        __syncthreads();
    }
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
    // 8); row 64 stays zero and pads the quadrant lists.
    __shared__ __align__(16) float table[(64 + 1) * REC];
    __shared__ __align__(16) uint8_t lists[ZCH][4][64];
    __shared__ float2 stage[ZST][64];
    const int64_t nw = (int64_t)nbx * nby * nseg;
    int64_t wid = xcd_remap(blockIdx.x, nw);
    const int seg = (int)(wid % nseg);
    wid /= nseg;
    const int by = (int)(wid % nby), bx = (int)(wid / nby);
    const int z0 = seg * zseg, zend = min(z0 + zseg, n2);
    const int lane = threadIdx.x, grp = lane >> 4;
    const int cxl = lane_cx(lane), cyl = lane_cy(lane);
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    if (lane < REC) table[64 * REC + lane] = 0.f;
    const int bxm = bx == 0 ? nbx - 1 : bx - 1, bym = by == 0 ? nby - 1 : by - 1;
    const int blk[NR] = {bx * nby + by, bxm * nby + by, bx * nby + bym, bxm * nby + bym};
    const int clo[NR] = {0, 2, 1, 2}, chi[NR] = {3, 3, 2, 2};
    float wre[W], wim[W];
#pragma unroll
    for (int a = 0; a < W; ++a) wre[a] = wim[a] = 0.f;
    int zw = z0 - (W - 1);  // z of window cell 0
    for (int zc = z0 - (W - 1); zc < zend; zc += ZCH) {
        int pf[ZCH * NR + 1], rs[ZCH * NR];
        pf[0] = 0;
#pragma unroll
        for (int t = 0; t < ZCH; ++t) {
            const int z = zc + t;
            const int zz = z < 0 ? z + n2 : z;
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                const int i = t * NR + r;
                int st = 0, cnt = 0;
                if (z < zend) {
                    const int64_t kb = ((int64_t)blk[r] * n2 + zz) * 4;
                    st = zstart[kb + clo[r]];
                    cnt = zstart[kb + chi[r] + 1] - st;
                }
                rs[i] = st;
                pf[i + 1] = pf[i] + cnt;
            }
        }
        const int tot = pf[ZCH * NR];
        for (int bat = 0; bat < tot; bat += 64) {
            const int nb = min(64, tot - bat);
            __syncthreads();
            reinterpret_cast<uint32_t *>(lists)[lane] = 0x40404040u;
            reinterpret_cast<uint32_t *>(lists)[lane + 64] = 0x40404040u;
            const bool valid = lane < nb;
            int tsel = -1, touch = 0;
            if (valid) {
                const int e = bat + lane;
                int i = 0;
#pragma unroll
                for (int q = 1; q < ZCH * NR; ++q) i += (e >= pf[q]) ? 1 : 0;
                int st = rs[0], p0 = pf[0];
#pragma unroll
                for (int q = 1; q < ZCH * NR; ++q)
                    if (q == i) {
                        st = rs[q];
                        p0 = pf[q];
                    }
                tsel = i / NR;
                const int64_t j = (int64_t)st + (e - p0);
                // first tap relative to this block: the word's in-block cell,
                // minus 8 for points of the -x / -y neighbour blocks
                const uint32_t wd = word[j];
                const int r = i % NR;
                const int ox = (int)((wd >> kZsKeyBits) & 7u) - ((r & 1) ? ZB : 0);
                const int oy = (int)((wd >> (kZsKeyBits + 3)) & 7u) - ((r & 2) ? ZB : 0);
                const float fx = frs.p[0][j], fy = frs.p[1][j], fz = frs.p[2][j];
                float2 cv = perm ? c[perm[j]] : c[j];
                if (pre) {
                    const float2 pv = pre[j];
                    cv = make_float2(cv.x * pv.x - cv.y * pv.y, cv.x * pv.y + cv.y * pv.x);
                }
                float4 *rec = reinterpret_cast<float4 *>(table + lane * REC);
                float wx[ZB], wy[ZB], wz[ZB];
#pragma unroll
                for (int q = 0; q < ZB; ++q) {
                    const int ax = q - ox, ay = q - oy;
                    wx[q] = ((unsigned)ax < (unsigned)W) ? es_weight((float)ax - fx, bl2e, inv_hw) : 0.f;
                    wy[q] = ((unsigned)ay < (unsigned)W) ? es_weight((float)ay - fy, bl2e, inv_hw) : 0.f;
                    wz[q] = q < W ? es_weight((float)q - fz, bl2e, inv_hw) : 0.f;
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
                    const bool mine = tsel == t && ((touch >> q) & 1);
                    const uint64_t bq = __ballot(mine);
                    cnt[t][q] = __popcll(bq);
                    if (mine) lists[t][q][__popcll(bq & lt_mask)] = (uint8_t)lane;
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
                const uint32_t *lw = reinterpret_cast<const uint32_t *>(lists[t][grp]);
                for (int it = 0; it < nit; it += UNR) {
                    const uint32_t pk = lw[it >> 2];
                    float vr[UNR], vi[UNR], wzz[UNR][W];
#pragma unroll
                    for (int u = 0; u < UNR; ++u) {
                        const float *rec = table + ((pk >> (8 * u)) & 0xffu) * REC;
                        const float2 wxc = *reinterpret_cast<const float2 *>(rec + 2 * cxl);
                        const float wyv = rec[16 + cyl];
                        vr[u] = wxc.x * wyv;
                        vi[u] = wxc.y * wyv;
#pragma unroll
                        for (int a = 0; a < W; ++a) wzz[u][a] = rec[24 + a];
                    }
#pragma unroll
                    for (int u = 0; u < UNR; ++u)
#pragma unroll
                        for (int a = 0; a < W; ++a) {
                            wre[a] = fmaf(vr[u], wzz[u][a], wre[a]);
                            wim[a] = fmaf(vi[u], wzz[u][a], wim[a]);
                        }
                }
            }
        }
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
            k_spread_zsweep<W><<<(unsigned)nw, 64, 0, a.s>>>(n0, n1, n2, nbx, nby, a.zseg, nseg,
                                                             bl2e, inv_hw, a.zstart, a.perm,
                                                             a.word, a.frs, a.c, a.pre, a.grid);
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
    return select_dim_w<ZLaunch>(3, g->w, a);
}

}  // extern "C"
