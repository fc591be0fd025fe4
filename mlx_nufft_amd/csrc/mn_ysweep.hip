// Owner-computes 2D spread ("y-sweep"): the 2D counterpart of the z-sweep.
// No atomics; every fine-grid cell is written exactly once.
//
// Layout. The grid (n0 x n1, n1 contiguous) is cut into blocks of 64
// consecutive x-columns. Each wavefront owns one block over a y-segment;
// lane l owns column 64 bx + l and keeps a W-cell complex window
// [y, y + W) of it in VGPRs. The wave walks y upwards: at each y it adds
// every point whose first tap is at y and whose footprint touches the
// block, then cell y is complete, is staged in LDS (so stores run along y)
// and the window shifts by one cell.
//
// Point order. Points are sorted by key (bx*n1 + y)*2 + reach, where bx, y
// come from the first tap and reach says whether the footprint crosses into
// the next block. Block b takes its own points (both reach values) and the
// reaching points of block b - 1: two contiguous key ranges per y, found
// through ystart (the first sorted index of each key). The sorted word
// carries the first tap's column within its block above the key.
//
// Per batch of up to 64 points of one y, a lane-per-point prologue builds a
// table row: the point's x-weights times its strength for the 16 columns of
// the two 8-column groups its footprint can touch (W <= 8), each group's
// 8 slots followed by the W y-weights. Per group, a list holds the byte
// offsets of the slot runs of the points touching it; the group's 8 lanes
// walk the list, each point costing 2*W FMAs per lane. Vectors of a batch
// are independent rows of the launch grid.
//
// The cursor (mn_cursor.h) walks groups of two y-steps; batches take up to
// 64 consecutive points of a group, with lists per y-step. Loads are issued
// by every lane outside any branch and the batch loop is unrolled three
// ways, so the words / fractions / perm of batch k + 2 and the strengths of
// batch k + 1 are in flight while batch k is built and swept.
//
// ref: nd.py:492-579 (the reference's output-driven spread this replaces),
// nd.py:683-742 (its batched spread), nd.py:298-372 (bin sort).
#include "mn_common.h"
#include "mn_cursor.h"

namespace mn {
namespace {

constexpr int YB = kYsBlock;  // columns per block (one per lane)
constexpr int YG = 8;         // lanes (columns) per group
constexpr int NG = YB / YG;   // groups per block
constexpr int YST = 4;        // y-cells staged in LDS per store
constexpr int YREC = 52;      // floats per table row (48 used; the pad spreads rows over banks)
constexpr int YRUN = 24;      // floats per group run: 8 complex slots + 8 y-weights

// Stage the finished cell of each column; every YST cells (or at the segment
// end) the wave writes them out, YST consecutive lanes per column storing
// YST consecutive y.
__device__ __forceinline__ void ys_store_stage(float2 (*stage)[64], float2 *__restrict__ grid,
                                               int lane, int s, int yw, int n1, int bx, float wr,
                                               float wi, bool last) {
    stage[s][lane] = make_float2(wr, wi);
    if (s == YST - 1 || last) {
        __syncthreads();
        const int yb = yw - s, ny = s + 1;
        for (int colb = 0; colb < 64; colb += 64 / YST) {
            const int col = colb + lane / YST, yo = lane % YST;
            if (yo < ny) grid[(int64_t)(YB * bx + col) * n1 + yb + yo] = stage[yo][col];
        }
        __syncthreads();
    }
}

constexpr int NRY = 2;  // key ranges per y: own block (both classes), -x neighbour (reaching)
constexpr int YZ = 2;   // y-steps per cursor group
constexpr int NQY = YZ * NRY;

// The bounds of the key ranges (SweepCursor fetch): range i = (y-step i / 2,
// source i % 2) of the group starting at yc. Source 0 is the block's own
// points, keys (bx n1 + y) * 2 + {0, 1}; source 1 is the -x neighbour's
// reaching points, key (bxm n1 + y) * 2 + 1. Every lane loads (key 0 for
// lanes without a range), outside any branch.
struct YFetch {
    int bx, dbx, n1, yend, nq;  // dbx = bxm - bx (the source is chosen by arithmetic)
    const int32_t *ystart;
    __device__ __forceinline__ int2 operator()(int yc, int lane) const {
        const int r = lane % NRY, y = yc + lane / NRY;
        const bool ok = lane < nq && y < yend;
        const int yy = y < 0 ? y + n1 : y;
        const int64_t kb = ok ? ((int64_t)(bx + r * dbx) * n1 + yy) * 2 : 0;
        const int st = ystart[kb + (ok ? r : 0)], en = ystart[kb + (ok ? 2 : 0)];
        return make_int2(ok ? st : 0, ok ? en : 0);
    }
};

// One lane's point of a batch, its loads issued (the strength, which needs
// src, is gathered one batch later).
struct YPoint {
    int yc, nb;        // the batch's group and size (uniform; nb = 0: done)
    bool valid;
    int tsel, r;       // y-step within the group and source
    uint32_t wd, src;  // sorted word; index of the strength in c
    float fx, fy;
};

// The next batch, its loads issued by every lane (an idle lane reads element
// 0) outside any branch, so the compiler can wait for exactly the loads a
// later use needs.
__device__ __forceinline__ YPoint yp_next(SweepCursor &k, const YFetch yf, int lane,
                                          SweepRanges<NQY> &rg, uint8_t *qidx,
                                          const uint32_t *__restrict__ perm,
                                          const uint32_t *__restrict__ word,
                                          const float *__restrict__ fx,
                                          const float *__restrict__ fy) {
    const SweepBatch sb = sweep_next<NQY, YZ>(k, yf.yend, rg, qidx, lane, yf);
    YPoint q;
    q.yc = sb.zc;
    q.nb = sb.nb;
    q.valid = sb.valid;
    q.tsel = sb.valid ? sb.range / NRY : -1;
    q.r = sb.range % NRY;
    const uint32_t j = sb.j;
    q.wd = word[j];
    q.fx = fx[j];
    q.fy = fy[j];
    const uint32_t pj = (perm ? perm : word)[j];
    q.src = perm ? pj : j;
    return q;
}

template <int W>
__global__ __launch_bounds__(64) void k_spread_ysweep(int n1, int nbx, int yseg, int nseg,
                                                      float bl2e, int64_t P,
                                                      const int32_t *__restrict__ ystart,
                                                      const uint32_t *__restrict__ perm,
                                                      const uint32_t *__restrict__ word,
                                                      const float *__restrict__ fx,
                                                      const float *__restrict__ fy,
                                                      const float2 *__restrict__ c,
                                                      float2 *__restrict__ grid, int64_t gsz) {
    __shared__ __align__(16) float table[(64 + 1) * YREC];
    __shared__ __align__(16) uint16_t lists[YZ][NG][64];
    __shared__ float2 stage[YST][64];
    __shared__ SweepRanges<NQY> rg;
    __shared__ uint8_t qidx[64];
    constexpr uint32_t kPad = 64u * YREC * 4u;  // byte offset of the zero row
    const int vec = blockIdx.y;
    c += (int64_t)vec * P;
    grid += (int64_t)vec * gsz;
    const int wid = (int)xcd_remap(blockIdx.x, (int64_t)nbx * nseg);
    const int seg = wid % nseg, bx = wid / nseg;
    const int bxm = bx == 0 ? nbx - 1 : bx - 1;
    const int y0 = seg * yseg, yend = min(y0 + yseg, n1);
    const int lane = threadIdx.x, grp = lane / YG, slot = lane % YG;
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    if (lane < YREC) table[64 * YREC + lane] = 0.f;
    float wre[W], wim[W];
#pragma unroll
    for (int a = 0; a < W; ++a) wre[a] = wim[a] = 0.f;
    int yw = y0 - (W - 1);  // y of window cell 0

    // Window cell 0 moves up by one: cell yw is complete (staged and stored
    // if this segment owns it).
    auto step = [&]() {
        if (yw >= y0)
            ys_store_stage(stage, grid, lane, (yw - y0) % YST, yw, n1, bx, wre[0], wim[0],
                           yw == yend - 1);
#pragma unroll
        for (int a = 0; a < W - 1; ++a) {
            wre[a] = wre[a + 1];
            wim[a] = wim[a + 1];
        }
        wre[W - 1] = wim[W - 1] = 0.f;
        ++yw;
    };

    // Build and sweep one batch p whose strengths are cp.
    auto process = [&](const YPoint &p, const float2 cp) __attribute__((always_inline)) {
        __syncthreads();
#pragma unroll
        for (int k = 0; k < YZ * NG * 32; k += 64)
            reinterpret_cast<uint32_t *>(lists)[k + lane] = kPad | (kPad << 16);
        int g0 = -1, touch2 = 0;
        if (p.valid) {
            // first tap relative to this block (-64 for the -x neighbour's points)
            const int ox = (int)(p.wd >> kYsKeyBits) - (p.r == 1 ? YB : 0);
            g0 = max(ox, 0) / YG;
            touch2 = (g0 + 1 < NG && YG * (g0 + 1) < ox + W) ? 1 : 0;
            float *rec = table + lane * YREC;
            constexpr float ih = 2.0f / W;
            const float sx = ((float)(YG * g0 - ox) - p.fx) * ih, sy = p.fy * ih;
            float wy[8];
#pragma unroll
            for (int a = 0; a < 8; ++a) wy[a] = a < W ? es_weight_z((float)a * ih - sy, bl2e) : 0.f;
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                float4 *run = reinterpret_cast<float4 *>(rec + r * YRUN);
#pragma unroll
                for (int q = 0; q < YG; q += 2) {
                    // columns YG*g0 + s, s = YG*r + q (+1): tap s + YG*g0 - ox
                    const int s = YG * r + q, a0 = YG * g0 + s - ox;
                    const float e0 = es_weight_z((float)s * ih + sx, bl2e);
                    const float e1 = es_weight_z((float)(s + 1) * ih + sx, bl2e);
                    const float w0 = (unsigned)a0 < (unsigned)W ? e0 : 0.f;
                    const float w1 = (unsigned)(a0 + 1) < (unsigned)W ? e1 : 0.f;
                    run[q / 2] = make_float4(cp.x * w0, cp.y * w0, cp.x * w1, cp.y * w1);
                }
                run[4] = make_float4(wy[0], wy[1], wy[2], wy[3]);
                run[5] = make_float4(wy[4], wy[5], wy[6], wy[7]);
            }
        }
        // per y-step and group: the batch runs that touch it, in order
        int cnt[YZ][NG];
#pragma unroll
        for (int t = 0; t < YZ; ++t)
#pragma unroll
            for (int q = 0; q < NG; ++q) {
                const bool mine = p.tsel == t;
                const bool first = mine && q == g0;
                const bool second = mine && touch2 && q == g0 + 1;
                const uint64_t bq = __ballot(first || second);
                cnt[t][q] = __popcll(bq);
                if (first || second)
                    lists[t][q][__popcll(bq & lt_mask)] =
                        (uint16_t)(lane * YREC * 4 + (second ? YRUN * 4 : 0));
            }
        __syncthreads();
        const char *tb = reinterpret_cast<const char *>(table);
#pragma unroll
        for (int t = 0; t < YZ; ++t) {
            int nit = cnt[t][0];
#pragma unroll
            for (int q = 1; q < NG; ++q) nit = max(nit, cnt[t][q]);
            if (nit == 0) continue;
            // the window moves to this step's y: usually one cell, as
            // straight-line code (a loop that stores makes the compiler wait
            // for every outstanding load before it)
            const int yt = p.yc + t;
            if (yw < yt) {
                step();
                while (yw < yt) step();
            }
            const uint16_t *lq = lists[t][grp];
            for (int it = 0; it < nit; ++it) {
                const char *run = tb + lq[it];
                const float2 v = *reinterpret_cast<const float2 *>(run + 8 * slot);
                const float4 z0 = *reinterpret_cast<const float4 *>(run + 64);
                float wz[8] = {z0.x, z0.y, z0.z, z0.w, 0.f, 0.f, 0.f, 0.f};
                if constexpr (W > 4) {
                    const float4 z1 = *reinterpret_cast<const float4 *>(run + 80);
                    wz[4] = z1.x, wz[5] = z1.y, wz[6] = z1.z, wz[7] = z1.w;
                }
#pragma unroll
                for (int a = 0; a < W; ++a) {
                    wre[a] = fmaf(v.x, wz[a], wre[a]);
                    wim[a] = fmaf(v.y, wz[a], wim[a]);
                }
            }
        }
    };

    // The batch loop, unrolled three ways with rotating names (A, B, C) so
    // that no register still being loaded is copied (a copy would wait for
    // it): each stage issues the loads of the batch two ahead, gathers the
    // strengths of the next one, then builds and sweeps the current one.
    const YFetch yf{bx, bxm - bx, n1, yend, NQY, ystart};
    SweepCursor cur;
    cur.pzc = INT32_MIN;
    sweep_load<NQY, YZ>(cur, y0 - (W - 1), rg, lane, yf);
    YPoint pa = yp_next(cur, yf, lane, rg, qidx, perm, word, fx, fy);
    float2 ca = c[pa.src];  // idle lanes read c[perm[0]]: their rows are never used
    YPoint pb = yp_next(cur, yf, lane, rg, qidx, perm, word, fx, fy);
    YPoint pc;
    float2 cb, cc;
    for (;;) {
        if (pa.nb == 0) break;
        pc = yp_next(cur, yf, lane, rg, qidx, perm, word, fx, fy);
        cb = c[pb.src];
        process(pa, ca);
        if (pb.nb == 0) break;
        pa = yp_next(cur, yf, lane, rg, qidx, perm, word, fx, fy);
        cc = c[pc.src];
        process(pb, cb);
        if (pc.nb == 0) break;
        pb = yp_next(cur, yf, lane, rg, qidx, perm, word, fx, fy);
        ca = c[pa.src];
        process(pc, cc);
    }
    while (yw < yend) step();  // drain the window up to the segment end
}

struct YsArgs {
    int n1, nbx, yseg, nseg;
    float bl2e;
    int64_t P, B, gsz;
    const int32_t *ystart;
    const uint32_t *perm, *word;
    const float *fx, *fy;
    const float2 *c;
    float2 *grid;
    hipStream_t s;
};

template <int W>
int ys_launch(const YsArgs &a) {
    const dim3 blocks((unsigned)(a.nbx * a.nseg), (unsigned)a.B);
    k_spread_ysweep<W><<<blocks, 64, 0, a.s>>>(a.n1, a.nbx, a.yseg, a.nseg, a.bl2e, a.P, a.ystart,
                                               a.perm, a.word, a.fx, a.fy, a.c, a.grid, a.gsz);
    MN_LAUNCH_CHECK("spread_ysweep");
    return MN_OK;
}

}  // namespace

int ysweep_check(const mn_bins *g) {
    MN_REQUIRE(g != nullptr && g->dim == 2, "ysweep: 2D geometry required");
    MN_REQUIRE(g->w >= 2 && g->w <= YG, "ysweep: kernel width must be in [2, 8]");
    MN_REQUIRE(g->n[0] % YB == 0 && g->n[0] >= 2 * YB, "ysweep: n0 must be a multiple of 64, >= 128");
    MN_REQUIRE(g->n[1] >= g->w && g->n[1] < (int64_t(1) << 24), "ysweep: n1 out of range");
    MN_REQUIRE(ysweep_nkeys(g) <= (int64_t(1) << kYsKeyBits), "ysweep: key space above 2^26");
    return MN_OK;
}

int64_t ysweep_nkeys(const mn_bins *g) { return (g->n[0] / YB) * g->n[1] * 2; }

}  // namespace mn

using namespace mn;

extern "C" {

int64_t mn_ysweep_nkeys(const mn_bins *g) {
    clear_error();
    if (ysweep_check(g)) return -1;
    return ysweep_nkeys(g);
}

int mn_ysweep_starts(const mn_bins *g, int64_t P, const uint32_t *sorted_word, int32_t *ystart,
                     mn_stream_t stream) {
    clear_error();
    int rc = ysweep_check(g);
    if (rc) return rc;
    MN_REQUIRE(P >= 1 && P < (int64_t(1) << 31), "ysweep starts: P must be in [1, 2^31)");
    MN_REQUIRE(sorted_word && ystart, "ysweep starts: NULL pointer");
    return key_starts(sorted_word, P, ysweep_nkeys(g), kYsKeyMask, ystart, as_stream(stream));
}

int mn_spread_ysweep(const mn_bins *g, float beta, int64_t P, int64_t B, int yseg,
                     const int32_t *ystart, const uint32_t *perm, const uint32_t *sorted_word,
                     const float *const frs[2], const void *c, void *grid, mn_stream_t stream) {
    clear_error();
    int rc = ysweep_check(g);
    if (rc) return rc;
    MN_REQUIRE(P >= 1 && P < (int64_t(1) << 31), "ysweep spread: P must be in [1, 2^31)");
    MN_REQUIRE(B >= 1 && B <= 65535, "ysweep spread: B must be in [1, 65535]");
    MN_REQUIRE(yseg >= 1, "ysweep spread: yseg must be >= 1");
    MN_REQUIRE(ystart && sorted_word && frs && frs[0] && frs[1] && c && grid,
               "ysweep spread: NULL pointer");
    YsArgs a{};
    a.n1 = (int)g->n[1];
    a.nbx = (int)(g->n[0] / YB);
    a.yseg = yseg;
    a.nseg = (int)((g->n[1] + yseg - 1) / yseg);
    MN_REQUIRE((int64_t)a.nbx * a.nseg < (int64_t(1) << 31), "ysweep spread: too many blocks");
    a.bl2e = (float)(beta * 1.4426950408889634);
    a.P = P;
    a.B = B;
    a.gsz = g->n[0] * g->n[1];
    a.ystart = ystart;
    a.perm = perm;
    a.word = sorted_word;
    a.fx = frs[0];
    a.fy = frs[1];
    a.c = static_cast<const float2 *>(c);
    a.grid = static_cast<float2 *>(grid);
    a.s = as_stream(stream);
    switch (g->w) {
        case 2: return ys_launch<2>(a);
        case 3: return ys_launch<3>(a);
        case 4: return ys_launch<4>(a);
        case 5: return ys_launch<5>(a);
        case 6: return ys_launch<6>(a);
        case 7: return ys_launch<7>(a);
        case 8: return ys_launch<8>(a);
    }
    set_error("ysweep spread: kernel width must be in [2, 8]");
    return MN_EINVAL;
}

}  // extern "C"
