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
// table row: for each of the two 8-column groups its footprint can touch
// (W <= 8), a run of the group's 8 x-weights, the W y-weights and the
// point's strengths in the wave's VB vectors. Per group, a list holds the
// byte offsets of the runs of the points touching it; the group's 8 lanes
// walk the list, each point costing, per vector, the strength times the
// lane's x-weight and 2*W FMAs into that vector's window. One wave carries
// VB vectors (a group of the batch's vectors per launch-grid row), so the
// cursor, the loads, the ES weights and the lists are shared by all of
// them; each vector's arithmetic is the same as with VB = 1.
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
// floats per group run: 8 x-weights, 8 y-weights, VB complex strengths,
// padded to a multiple of 4 so that every run is 16-byte aligned
template <int VB>
constexpr int yrun() { return (16 + 2 * VB + 3) / 4 * 4; }
// floats per table row: two runs, padded to 4 mod 8 dwords so that the 16-byte
// row stores of neighbouring lanes spread over the LDS banks
template <int VB>
constexpr int yrec() { return (2 * yrun<VB>()) % 8 == 4 ? 2 * yrun<VB>() : 2 * yrun<VB>() + 4; }

// Stage the finished cell of each column of every vector; every YST cells
// (or at the segment end) the wave writes them out, YST consecutive lanes
// per column storing YST consecutive y.
template <int VB>
__device__ __forceinline__ void ys_store_stage(float2 (*stage)[YST][64], float2 *__restrict__ grid,
                                               int64_t gsz, int nv, int lane, int s, int yw, int n1,
                                               int bx, const float *wr, const float *wi,
                                               bool last) {
#pragma unroll
    for (int v = 0; v < VB; ++v) stage[v][s][lane] = make_float2(wr[v], wi[v]);
    if (s == YST - 1 || last) {
        __syncthreads();
        const int yb = yw - s, ny = s + 1;
#pragma unroll
        for (int v = 0; v < VB; ++v) {
            if (v >= nv) break;
            for (int colb = 0; colb < 64; colb += 64 / YST) {
                const int col = colb + lane / YST, yo = lane % YST;
                if (yo < ny)
                    grid[v * gsz + (int64_t)(YB * bx + col) * n1 + yb + yo] = stage[v][yo][col];
            }
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

template <int W, int VB>
__global__ __launch_bounds__(64) void k_spread_ysweep(int n1, int nbx, int yseg, int nseg,
                                                      float bl2e, int64_t P, int64_t B,
                                                      const int32_t *__restrict__ ystart,
                                                      const uint32_t *__restrict__ perm,
                                                      const uint32_t *__restrict__ word,
                                                      const float *__restrict__ fx,
                                                      const float *__restrict__ fy,
                                                      const float2 *__restrict__ c,
                                                      float2 *__restrict__ grid, int64_t gsz) {
    constexpr int YRUN = yrun<VB>(), YREC = yrec<VB>();
    __shared__ __align__(16) float table[(64 + 1) * YREC];
    __shared__ __align__(16) uint16_t lists[YZ][NG][64];
    __shared__ float2 stage[VB][YST][64];
    __shared__ SweepRanges<NQY> rg;
    __shared__ uint8_t qidx[64];
    constexpr uint32_t kPad = 64u * YREC * 4u;  // byte offset of the zero row
    static_assert(kPad + YREC * 4u < 65536u, "list offsets are 16-bit");
    const int64_t v0 = (int64_t)blockIdx.y * VB;
    const int nv = (int)min((int64_t)VB, B - v0);  // vectors of this wave (>= 1)
    c += v0 * P;
    grid += v0 * gsz;
    const int wid = (int)xcd_remap(blockIdx.x, (int64_t)nbx * nseg);
    const int seg = wid % nseg, bx = wid / nseg;
    const int bxm = bx == 0 ? nbx - 1 : bx - 1;
    const int y0 = seg * yseg, yend = min(y0 + yseg, n1);
    const int lane = threadIdx.x, grp = lane / YG, slot = lane % YG;
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int i = lane; i < YREC; i += 64) table[64 * YREC + i] = 0.f;
    float wre[VB][W], wim[VB][W];
#pragma unroll
    for (int v = 0; v < VB; ++v)
#pragma unroll
        for (int a = 0; a < W; ++a) wre[v][a] = wim[v][a] = 0.f;
    int yw = y0 - (W - 1);  // y of window cell 0

    // Window cell 0 moves up by one: cell yw is complete (staged and stored
    // if this segment owns it).
    auto step = [&]() {
        if (yw >= y0) {
            float c0r[VB], c0i[VB];
#pragma unroll
            for (int v = 0; v < VB; ++v) c0r[v] = wre[v][0], c0i[v] = wim[v][0];
            ys_store_stage<VB>(stage, grid, gsz, nv, lane, (yw - y0) % YST, yw, n1, bx, c0r, c0i,
                               yw == yend - 1);
        }
#pragma unroll
        for (int v = 0; v < VB; ++v) {
#pragma unroll
            for (int a = 0; a < W - 1; ++a) {
                wre[v][a] = wre[v][a + 1];
                wim[v][a] = wim[v][a + 1];
            }
            wre[v][W - 1] = wim[v][W - 1] = 0.f;
        }
        ++yw;
    };

    // Build and sweep one batch p whose strengths (per vector) are cp.
    auto process = [&](const YPoint &p, const float2 *cp) __attribute__((always_inline)) {
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
                float *run = rec + r * YRUN;
                float wx[YG];
#pragma unroll
                for (int q = 0; q < YG; ++q) {
                    // column YG*g0 + s, s = YG*r + q: tap s + YG*g0 - ox
                    const int s = YG * r + q, a0 = YG * g0 + s - ox;
                    const float e = es_weight_z((float)s * ih + sx, bl2e);
                    wx[q] = (unsigned)a0 < (unsigned)W ? e : 0.f;
                }
                float4 *r4 = reinterpret_cast<float4 *>(run);
                r4[0] = make_float4(wx[0], wx[1], wx[2], wx[3]);
                r4[1] = make_float4(wx[4], wx[5], wx[6], wx[7]);
                r4[2] = make_float4(wy[0], wy[1], wy[2], wy[3]);
                r4[3] = make_float4(wy[4], wy[5], wy[6], wy[7]);
                float2 *r2 = reinterpret_cast<float2 *>(run + 16);
#pragma unroll
                for (int v = 0; v < VB; ++v) r2[v] = cp[v];
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
                const float *run = reinterpret_cast<const float *>(tb + lq[it]);
                const float wxs = run[slot];
                const float4 z0 = *reinterpret_cast<const float4 *>(run + 8);
                float wz[8] = {z0.x, z0.y, z0.z, z0.w, 0.f, 0.f, 0.f, 0.f};
                if constexpr (W > 4) {
                    const float4 z1 = *reinterpret_cast<const float4 *>(run + 12);
                    wz[4] = z1.x, wz[5] = z1.y, wz[6] = z1.z, wz[7] = z1.w;
                }
                const float2 *cv = reinterpret_cast<const float2 *>(run + 16);
#pragma unroll
                for (int v = 0; v < VB; ++v) {
                    const float2 cw = cv[v];
                    const float vr = cw.x * wxs, vi = cw.y * wxs;
#pragma unroll
                    for (int a = 0; a < W; ++a) {
                        wre[v][a] = fmaf(vr, wz[a], wre[v][a]);
                        wim[v][a] = fmaf(vi, wz[a], wim[v][a]);
                    }
                }
            }
        }
    };

    // Strengths of one batch in every vector of the wave (vectors past nv
    // read the last valid one; their windows are never stored).
    auto gather = [&](const YPoint &p, float2 *cp) __attribute__((always_inline)) {
#pragma unroll
        for (int v = 0; v < VB; ++v) cp[v] = c[(int64_t)min(v, nv - 1) * P + p.src];
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
    float2 ca[VB], cb[VB], cc[VB];
    gather(pa, ca);  // idle lanes read c[perm[0]]: their rows are never used
    YPoint pb = yp_next(cur, yf, lane, rg, qidx, perm, word, fx, fy);
    YPoint pc;
    for (;;) {
        if (pa.nb == 0) break;
        pc = yp_next(cur, yf, lane, rg, qidx, perm, word, fx, fy);
        gather(pb, cb);
        process(pa, ca);
        if (pb.nb == 0) break;
        pa = yp_next(cur, yf, lane, rg, qidx, perm, word, fx, fy);
        gather(pc, cc);
        process(pb, cb);
        if (pc.nb == 0) break;
        pb = yp_next(cur, yf, lane, rg, qidx, perm, word, fx, fy);
        gather(pa, ca);
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

// Vectors per wave: the largest of 8, 4, 2, 1 not above B (measured at
// 2048^2, 1e7 points, w = 7, B = 8: 2.19 ms at VB = 8 with 64-row segments,
// 2.3-2.4 ms at VB = 2 or 4, 5.5 ms at VB = 1).
inline int ys_vb(int64_t B) { return B >= 8 ? 8 : (B >= 4 ? 4 : (B >= 2 ? 2 : 1)); }

template <int W, int VB>
int ys_launch_vb(const YsArgs &a) {
    const dim3 blocks((unsigned)(a.nbx * a.nseg), (unsigned)((a.B + VB - 1) / VB));
    k_spread_ysweep<W, VB><<<blocks, 64, 0, a.s>>>(a.n1, a.nbx, a.yseg, a.nseg, a.bl2e, a.P, a.B,
                                                   a.ystart, a.perm, a.word, a.fx, a.fy, a.c,
                                                   a.grid, a.gsz);
    MN_LAUNCH_CHECK("spread_ysweep");
    return MN_OK;
}

template <int W>
int ys_launch(const YsArgs &a) {
    switch (ys_vb(a.B)) {
        case 8: return ys_launch_vb<W, 8>(a);
        case 4: return ys_launch_vb<W, 4>(a);
        case 2: return ys_launch_vb<W, 2>(a);
        default: return ys_launch_vb<W, 1>(a);
    }
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
