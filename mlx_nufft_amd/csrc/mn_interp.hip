// Interpolation (type-2 core, and the type-3 target gather) on LDS tiles.
//
// One 256-thread workgroup per subproblem loads the bin's padded tile of the
// fine grid (m + w - 1 cells per dim, periodic wrap) into LDS once, with
// rows along the contiguous last dim; then the lanes gather the points from
// LDS: w^dim complex taps per point, summed along the last dim first and
// weighted by the product of the other dims' ES weights. In 3D a pair of
// neighbouring lanes shares a point (alternate x-planes, one shuffle to add
// them): a bin holds about 76 points at 2e7 points on 512^3, so one lane per
// point left most lanes idle (measured 1.92 -> 1.72-1.80 ms there). The result is
// scattered to caller order (out[perm[j]]), optionally times a sorted-order
// multiplier (the type-3 post factor).
// ref: nd.py:974-1073 (OD gather), nd.py:908-972 (GM gather),
// gpu_t3.py:653-693 (type-3 gather x post).
#include "mn_common.h"

#include <stdlib.h>

namespace mn {
namespace {

struct InterpArgs {
    const mn_bins *g;
    float beta;
    int64_t nsub;
    const int32_t *info;
    const uint32_t *perm;
    CI3s i1s;
    CF3s frs;
    const float2 *grid;
    const float2 *post;
    float2 *out;
    hipStream_t s;
};

__device__ __forceinline__ int wrap_tile_i(int v, int n) {
    v = wrap1(v, n);
    if (v >= n) v -= n;
    return v;
}

template <int DIM, int W>
__global__ __launch_bounds__(256) void k_interp_tiled(Geom g, float bl2e, float inv_hw,
                                                      int64_t nsub, const int32_t *__restrict__ info,
                                                      const uint32_t *__restrict__ perm, CI3s i1s,
                                                      CF3s frs, const float2 *__restrict__ grid,
                                                      const float2 *__restrict__ post,
                                                      float2 *__restrict__ out) {
    extern __shared__ float2 tile[];
    const int p1 = g.p[1], p2 = g.p[2];
    const int T = g.p[0] * p1 * p2;
    const int64_t sub = xcd_remap(blockIdx.x, nsub);
    const int bin = info[3 * sub], s0 = info[3 * sub + 1], cnt = info[3 * sub + 2];
    int b[3] = {0, 0, 0};
    {
        int rem = bin;
#pragma unroll
        for (int d = DIM - 1; d >= 0; --d) {
            b[d] = rem % g.nb[d];
            rem /= g.nb[d];
        }
    }
    const int o0 = b[0] * g.m[0] - W / 2;
    const int o1 = DIM >= 2 ? b[1] * g.m[1] - W / 2 : 0;
    const int o2 = DIM >= 3 ? b[2] * g.m[2] - W / 2 : 0;
    {
        // Tile cell q = (q0*p1 + q1)*p2 + q2, walked with a stride of nt as a
        // mixed-radix counter (no division per cell). Loads go out in batches
        // of LB cells per thread before any LDS write, so their latencies
        // overlap; bins whose padded tile lies inside the grid (uniform per
        // workgroup) skip the periodic wrap.
        constexpr int LB = 8;
        const int nt = blockDim.x;
        const int s2 = nt % p2, s12 = nt / p2, s1 = s12 % p1, s0 = s12 / p1;
        int q2 = threadIdx.x % p2, q1 = (threadIdx.x / p2) % p1, q0 = threadIdx.x / (p2 * p1);
        const bool inside = o0 >= 0 && o0 + g.p[0] <= g.n[0] && o1 >= 0 && o1 + p1 <= g.n[1] &&
                            o2 >= 0 && o2 + p2 <= g.n[2];
        const int64_t n12 = (int64_t)g.n[1] * g.n[2];
        for (int qb = threadIdx.x; qb < T; qb += nt * LB) {
            float2 v[LB];
#pragma unroll
            for (int b = 0; b < LB; ++b) {
                const int q = qb + b * nt;
                v[b] = make_float2(0.f, 0.f);
                if (q < T) {
                    int64_t idx;
                    if (inside) {
                        idx = (int64_t)(o0 + q0) * n12 + (int64_t)(o1 + q1) * g.n[2] + (o2 + q2);
                    } else {
                        const int g0 = wrap_tile_i(o0 + q0, g.n[0]);
                        const int g1 = DIM >= 2 ? wrap_tile_i(o1 + q1, g.n[1]) : 0;
                        const int g2 = DIM >= 3 ? wrap_tile_i(o2 + q2, g.n[2]) : 0;
                        idx = ((int64_t)g0 * g.n[1] + g1) * g.n[2] + g2;
                    }
                    v[b] = grid[idx];
                }
                q2 += s2;
                int c = q2 >= p2;
                q2 -= c ? p2 : 0;
                q1 += s1 + c;
                c = q1 >= p1;
                q1 -= c ? p1 : 0;
                q0 += s0 + c;
            }
#pragma unroll
            for (int b = 0; b < LB; ++b) {
                const int q = qb + b * nt;
                if (q < T) tile[q] = v[b];
            }
        }
    }
    __syncthreads();

    if constexpr (DIM == 3) {
        // The lanes of one tile read add the same tap offset to their
        // points' bases, so points whose bases agree modulo 32 float2 (the
        // 64 four-byte banks) collide. The subproblem's points are taken in
        // an order that deals them round-robin over 16 classes of base / 2
        // (a lane pair reads base and base + p1 p2 for its two x-planes):
        // round k holds the k-th point of every class that has one.
        constexpr int ORD_MAX = 1024;  // points per subproblem the reordering takes
        __shared__ uint16_t ord[ORD_MAX];
        __shared__ int rcnt[16];
        const bool use_ord = cnt <= ORD_MAX;
        if (use_ord) {
            if (threadIdx.x < 16) rcnt[threadIdx.x] = 0;
            __syncthreads();
            constexpr int NI = ORD_MAX / 256;
            int res[NI], rk[NI];
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int t = threadIdx.x + 256 * i;
                res[i] = rk[i] = 0;
                if (t < cnt && (int)blockDim.x == 256) {
                    const int64_t j = (int64_t)s0 + t;
                    int lc[3];
#pragma unroll
                    for (int d = 0; d < 3; ++d) {
                        int v = wrap1(i1s.p[d][j] + W / 2, g.n[d]);
                        if ((unsigned)v >= (unsigned)g.n[d]) v = pmod(v, g.n[d]);
                        lc[d] = v - b[d] * g.m[d];
                    }
                    res[i] = (((lc[0] * p1 + lc[1]) * p2 + lc[2]) >> 1) & 15;
                    rk[i] = atomicAdd(&rcnt[res[i]], 1);
                }
            }
            __syncthreads();
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int t = threadIdx.x + 256 * i;
                if (t < cnt && (int)blockDim.x == 256) {
                    int slot = 0;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int n = rcnt[r];
                        slot += min(n, rk[i]) + ((r < res[i] && n > rk[i]) ? 1 : 0);
                    }
                    ord[slot] = (uint16_t)t;
                }
            }
            __syncthreads();
        }
        const bool ordered = use_ord && (int)blockDim.x == 256;
        // two lanes per point (a pair of neighbouring lanes): lane h of the
        // pair sums the x-planes a0 = h, h + 2, ...; one shuffle adds them
        for (int t = threadIdx.x; t < 2 * cnt; t += blockDim.x) {
            const int pt = ordered ? (int)ord[t >> 1] : (t >> 1), h = t & 1;
            const int64_t j = (int64_t)s0 + pt;
            int loc[3];
            bool ok = true;
            float wt1[W], wt2[W];
#pragma unroll
            for (int d = 0; d < 3; ++d) {
                int v = wrap1(i1s.p[d][j] + W / 2, g.n[d]);
                if ((unsigned)v >= (unsigned)g.n[d]) v = pmod(v, g.n[d]);
                loc[d] = v - b[d] * g.m[d];
                ok = ok && (unsigned)loc[d] < (unsigned)g.m[d];
            }
            const float f0 = frs.p[0][j], f1 = frs.p[1][j], f2 = frs.p[2][j];
#pragma unroll
            for (int a = 0; a < W; ++a) {
                wt1[a] = es_weight((float)a - f1, bl2e, inv_hw);
                wt2[a] = es_weight((float)a - f2, bl2e, inv_hw);
            }
            float ar = 0.0f, ai = 0.0f;
            if (ok) {
#pragma unroll
                for (int k = 0; k < (W + 1) / 2; ++k) {
                    const int a0 = 2 * k + h;
                    if (a0 < W) {
                        const float w0 = es_weight((float)a0 - f0, bl2e, inv_hw);
                        float pr = 0.0f, pi = 0.0f;
#pragma unroll
                        for (int a1 = 0; a1 < W; ++a1) {
                            const int base = ((loc[0] + a0) * p1 + loc[1] + a1) * p2 + loc[2];
                            float sr = 0.0f, si = 0.0f;
#pragma unroll
                            for (int a2 = 0; a2 < W; ++a2) {
                                const float2 v = tile[base + a2];
                                sr = fmaf(v.x, wt2[a2], sr);
                                si = fmaf(v.y, wt2[a2], si);
                            }
                            pr = fmaf(sr, wt1[a1], pr);
                            pi = fmaf(si, wt1[a1], pi);
                        }
                        ar = fmaf(pr, w0, ar);
                        ai = fmaf(pi, w0, ai);
                    }
                }
            }
            ar += __shfl_xor(ar, 1, 64);
            ai += __shfl_xor(ai, 1, 64);
            if (h == 0) {
                float2 r = make_float2(ar, ai);
                if (post) {
                    const float2 pv = post[j];
                    r = make_float2(ar * pv.x - ai * pv.y, ar * pv.y + ai * pv.x);
                }
                out[perm[j]] = r;
            }
        }
        return;
    }
    for (int t = threadIdx.x; t < cnt; t += blockDim.x) {
        const int64_t j = (int64_t)s0 + t;
        float wt[DIM][W];
        int loc[3] = {0, 0, 0};
        bool ok = true;
#pragma unroll
        for (int d = 0; d < DIM; ++d) {
            int v = wrap1(i1s.p[d][j] + W / 2, g.n[d]);
            if ((unsigned)v >= (unsigned)g.n[d]) v = pmod(v, g.n[d]);
            loc[d] = v - b[d] * g.m[d];
            ok = ok && (unsigned)loc[d] < (unsigned)g.m[d];
            const float f = frs.p[d][j];
#pragma unroll
            for (int a = 0; a < W; ++a) wt[d][a] = es_weight((float)a - f, bl2e, inv_hw);
        }
        float ar = 0.0f, ai = 0.0f;
        if (ok) {
            if constexpr (DIM == 1) {
#pragma unroll
                for (int a0 = 0; a0 < W; ++a0) {
                    const float2 v = tile[loc[0] + a0];
                    ar = fmaf(v.x, wt[0][a0], ar);
                    ai = fmaf(v.y, wt[0][a0], ai);
                }
            } else if constexpr (DIM == 2) {
#pragma unroll
                for (int a0 = 0; a0 < W; ++a0) {
                    const int base = (loc[0] + a0) * p1 + loc[1];
                    float sr = 0.0f, si = 0.0f;
#pragma unroll
                    for (int a1 = 0; a1 < W; ++a1) {
                        const float2 v = tile[base + a1];
                        sr = fmaf(v.x, wt[1][a1], sr);
                        si = fmaf(v.y, wt[1][a1], si);
                    }
                    ar = fmaf(sr, wt[0][a0], ar);
                    ai = fmaf(si, wt[0][a0], ai);
                }
            } else {
#pragma unroll
                for (int a0 = 0; a0 < W; ++a0) {
#pragma unroll
                    for (int a1 = 0; a1 < W; ++a1) {
                        const int base = ((loc[0] + a0) * p1 + loc[1] + a1) * p2 + loc[2];
                        float sr = 0.0f, si = 0.0f;
#pragma unroll
                        for (int a2 = 0; a2 < W; ++a2) {
                            const float2 v = tile[base + a2];
                            sr = fmaf(v.x, wt[2][a2], sr);
                            si = fmaf(v.y, wt[2][a2], si);
                        }
                        const float w01 = wt[0][a0] * wt[1][a1];
                        ar = fmaf(sr, w01, ar);
                        ai = fmaf(si, w01, ai);
                    }
                }
            }
        }
        float2 r = make_float2(ar, ai);
        if (post) {
            const float2 pv = post[j];
            r = make_float2(ar * pv.x - ai * pv.y, ar * pv.y + ai * pv.x);
        }
        out[perm[j]] = r;
    }
}

// Direct gather (3D) for point sets that are sparse on their grid (the
// type-3 targets): no tile is staged; each point's w^3 taps are read straight
// from the grid through L1/L2. A group of w lanes shares one point, lane z of
// the group taking z-offset z of every (x, y) row, so one load instruction
// reads w contiguous cells for each of the wave's 64 / w points (a handful
// of cache lines per instruction, not one per lane). Each lane sums its
// column over the w^2 rows with the x and y weights, scales by its z weight,
// and the group's first lane adds the w partial sums (shuffles) and writes
// the point. A tile costs (m + w - 1)^3 cells per non-empty bin whatever
// the bin holds, so with about one point per bin this reads several times
// fewer bytes. Blocks are remapped so each XCD walks a contiguous run of
// sorted points (neighbours share rows in its L2).
constexpr int DI_THREADS = 256;

template <int W>
__global__ __launch_bounds__(DI_THREADS) void k_interp_direct(Geom g, float bl2e, float inv_hw,
                                                              int64_t P, int64_t nblk,
                                                              const uint32_t *__restrict__ perm,
                                                              CI3s i1s, CF3s frs,
                                                              const float2 *__restrict__ grid,
                                                              const float2 *__restrict__ post,
                                                              float2 *__restrict__ out) {
    constexpr int TPW = 64 / W;                   // points per wave
    constexpr int TPB = TPW * (DI_THREADS / 64);  // points per block
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int grp = lane / W, z = lane - grp * W;
    const int64_t j0 = xcd_remap(blockIdx.x, nblk) * TPB + (int64_t)wv * TPW;
    const int64_t j = j0 + grp;
    const bool live = grp < TPW && j < P;
    const int64_t jj = live ? j : 0;  // idle lanes read point 0 (P >= 1)
    const int n0 = g.n[0], n1 = g.n[1], n2 = g.n[2];
    const int i0 = i1s.p[0][jj], i1 = i1s.p[1][jj], i2 = i1s.p[2][jj];
    const float f0 = frs.p[0][jj], f1 = frs.p[1][jj], f2 = frs.p[2][jj];
    float w0[W], w1[W];
    int gy[W];
#pragma unroll
    for (int a = 0; a < W; ++a) {
        w0[a] = es_weight((float)a - f0, bl2e, inv_hw);
        w1[a] = es_weight((float)a - f1, bl2e, inv_hw);
        gy[a] = wrap_tile_i(i1 + a, n1);
    }
    const float wz = es_weight((float)z - f2, bl2e, inv_hw);
    const int gz = wrap_tile_i(i2 + z, n2);
    float ar = 0.0f, ai = 0.0f;
    // unrolled: the W x W loads stay in flight across x-planes (rolled, each
    // plane waited for its W loads)
#pragma unroll
    for (int a0 = 0; a0 < W; ++a0) {
        const int64_t gx = wrap_tile_i(i0 + a0, n0);
        const float2 *col = grid + gx * n1 * (int64_t)n2 + gz;
        float pr = 0.0f, pi = 0.0f;
#pragma unroll
        for (int a1 = 0; a1 < W; ++a1) {
            const float2 v = col[(int64_t)gy[a1] * n2];
            pr = fmaf(v.x, w1[a1], pr);
            pi = fmaf(v.y, w1[a1], pi);
        }
        ar = fmaf(pr, w0[a0], ar);
        ai = fmaf(pi, w0[a0], ai);
    }
    ar *= wz;
    ai *= wz;
    // group sum: lane grp*W adds the other W - 1 lanes of its group
    const int base = grp * W;
    float sr = ar, si = ai;
#pragma unroll
    for (int k = 1; k < W; ++k) {
        const int src = min(base + k, 63);
        const float xr = __shfl(ar, src, 64), xi = __shfl(ai, src, 64);
        sr += xr;
        si += xi;
    }
    if (live && z == 0) {
        float2 r = make_float2(sr, si);
        if (post) {
            const float2 pv = post[j];
            r = make_float2(sr * pv.x - si * pv.y, sr * pv.y + si * pv.x);
        }
        out[perm[j]] = r;
    }
}

template <int DIM, int W>
struct DirectInterpLaunch {
    static int run(const InterpArgs &a) {
        if constexpr (DIM != 3) {
            set_error("interp direct: 3D only");
            return MN_EINVAL;
        } else {
            Geom g = make_geom(a.g);
            const float bl2e = (float)(a.beta * 1.4426950408889634);
            const float inv_hw = (float)(2.0 / W);
            const int64_t P = a.nsub;  // the point count travels in nsub here
            constexpr int TPB = (64 / W) * (DI_THREADS / 64);
            const int64_t nblk = (P + TPB - 1) / TPB;
            k_interp_direct<W><<<(unsigned)nblk, DI_THREADS, 0, a.s>>>(
                g, bl2e, inv_hw, P, nblk, a.perm, a.i1s, a.frs, a.grid, a.post, a.out);
            MN_LAUNCH_CHECK("interp direct");
            return MN_OK;
        }
    }
};

int interp_threads() {
    static const int v = [] {
        const char *e = getenv("MN_INTERP_THREADS");
        const int n = e ? atoi(e) : 256;
        return (n == 64 || n == 128 || n == 256) ? n : 256;
    }();
    return v;
}

template <int DIM, int W>
struct InterpLaunch {
    static int run(const InterpArgs &a) {
        Geom g = make_geom(a.g);
        const float bl2e = (float)(a.beta * 1.4426950408889634);
        const float inv_hw = (float)(2.0 / W);
        const size_t lds = (size_t)tile_cells(a.g) * sizeof(float2);
        if (lds > (size_t)max_lds_per_block()) {
            set_error("interp: tile does not fit in LDS; use smaller bins");
            return MN_EINVAL;
        }
        if (a.nsub == 0) return MN_OK;
        auto kern = k_interp_tiled<DIM, W>;
        if (lds > 65536)
            MN_HIP_CHECK(hipFuncSetAttribute((const void *)kern,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        kern<<<(unsigned)a.nsub, interp_threads(), lds, a.s>>>(g, bl2e, inv_hw, a.nsub, a.info, a.perm, a.i1s,
                                                  a.frs, a.grid, a.post, a.out);
        MN_LAUNCH_CHECK("interp");
        return MN_OK;
    }
};

// ---------------------------------------------------------------------------
// z-streaming interpolation (3D): bins of 16 x 16 columns x 8 z-cells. One
// 256-thread workgroup owns a 16 x 16 column block over a run of consecutive
// z-bins and keeps an LDS window of the grid -- the block's columns plus the
// kernel halo, (16 + w - 1)^2 columns x (8 + w - 1) z-cells -- that slides
// along z: after a bin's points are interpolated, the window's last w - 1
// z-cells move to its front and the next 8 z-cells of every column, loaded
// into registers while the points were being interpolated, fill the rest.
// Every grid cell is read (16 + w - 1)^2 / 16^2 times (1.7x at w = 6)
// instead of the (m + w - 1)^3 / m^3 of independent tiles, and the loads
// overlap the gather. Points: one lane per point, as in k_interp_tiled.
constexpr int ZI_BX = 16, ZI_BY = 16, ZI_ZT = 8;
constexpr int ZI_THREADS = 256;

template <int W>
struct ZWin {
    static constexpr int PX = ZI_BX + W - 1, PY = ZI_BY + W - 1;
    static constexpr int NC = PX * PY;              // window columns
    static constexpr int ZW = ZI_ZT + W - 1;        // window depth
    static constexpr int ZP = ZW | 1;               // odd row pitch (LDS banks)
    static constexpr int NNEW = NC * ZI_ZT;         // cells per slide
    static constexpr int NPT = (NNEW + ZI_THREADS - 1) / ZI_THREADS;
    static constexpr int NKEEP = NC * (W - 1);      // cells kept per slide
    static constexpr int NKPT = (NKEEP + ZI_THREADS - 1) / ZI_THREADS;
    static constexpr size_t LDS = sizeof(float2) * NC * ZP;
};

template <int W>
__global__ __launch_bounds__(ZI_THREADS) void k_interp_zstream(
    Geom g, float bl2e, float inv_hw, int nseg, int segbins, const int32_t *__restrict__ bstart,
    const uint32_t *__restrict__ perm, CI3s i1s, CF3s frs, const float2 *__restrict__ grid,
    const float2 *__restrict__ post, float2 *__restrict__ out) {
    using Z = ZWin<W>;
    extern __shared__ float2 win[];
    const int nbx = g.nb[0], nby = g.nb[1], nbz = g.nb[2];
    int64_t wid = xcd_remap(blockIdx.x, (int64_t)nbx * nby * nseg);
    const int seg = (int)(wid % nseg);
    wid /= nseg;
    const int by = (int)(wid % nby), bx = (int)(wid / nby);
    const int bz0 = seg * segbins, bz1 = min(bz0 + segbins, nbz);
    if (bz0 >= bz1) return;  // whole workgroup
    const int tid = threadIdx.x;
    const int x0 = bx * ZI_BX - W / 2, y0 = by * ZI_BY - W / 2;
    const int64_t n12 = (int64_t)g.n[1] * g.n[2];
    // the full window of the first bin
    {
        const int zlo = bz0 * ZI_ZT - W / 2;
        for (int e = tid; e < Z::NC * Z::ZW; e += ZI_THREADS) {
            const int c = e / Z::ZW, q = e % Z::ZW;
            const int gx = wrap_tile_i(x0 + c / Z::PY, g.n[0]);
            const int gy = wrap_tile_i(y0 + c % Z::PY, g.n[1]);
            const int gz = wrap_tile_i(zlo + q, g.n[2]);
            win[c * Z::ZP + q] = grid[gx * n12 + (int64_t)gy * g.n[2] + gz];
        }
    }
    __syncthreads();
    float2 nxt[Z::NPT];
    for (int bz = bz0; bz < bz1; ++bz) {
        const bool more = bz + 1 < bz1;
        if (more) {  // the next 8 z-cells of every window column
            const int znew = bz * ZI_ZT - W / 2 + Z::ZW;
#pragma unroll
            for (int i = 0; i < Z::NPT; ++i) {
                const int e = tid + i * ZI_THREADS;
                if (e < Z::NNEW) {
                    const int c = e / ZI_ZT, q = e % ZI_ZT;
                    const int gx = wrap_tile_i(x0 + c / Z::PY, g.n[0]);
                    const int gy = wrap_tile_i(y0 + c % Z::PY, g.n[1]);
                    const int gz = wrap_tile_i(znew + q, g.n[2]);
                    nxt[i] = grid[gx * n12 + (int64_t)gy * g.n[2] + gz];
                }
            }
        }
        const int64_t bin = ((int64_t)bx * nby + by) * nbz + bz;
        const int s0 = bstart[bin], s1 = bstart[bin + 1];
        for (int tt = s0 + tid; tt < s1; tt += ZI_THREADS) {
            const int64_t j = tt;
            float wt[3][W];
            int loc[3];
            bool ok = true;
            const int org[3] = {bx * ZI_BX, by * ZI_BY, bz * ZI_ZT};
            const int lim[3] = {ZI_BX, ZI_BY, ZI_ZT};
#pragma unroll
            for (int d = 0; d < 3; ++d) {
                int v = wrap1(i1s.p[d][j] + W / 2, g.n[d]);
                if ((unsigned)v >= (unsigned)g.n[d]) v = pmod(v, g.n[d]);
                loc[d] = v - org[d];
                ok = ok && (unsigned)loc[d] < (unsigned)lim[d];
                const float f = frs.p[d][j];
#pragma unroll
                for (int a = 0; a < W; ++a) wt[d][a] = es_weight((float)a - f, bl2e, inv_hw);
            }
            float ar = 0.0f, ai = 0.0f;
            if (ok) {
#pragma unroll
                for (int a0 = 0; a0 < W; ++a0) {
#pragma unroll
                    for (int a1 = 0; a1 < W; ++a1) {
                        const int base = ((loc[0] + a0) * Z::PY + loc[1] + a1) * Z::ZP + loc[2];
                        float sr = 0.0f, si = 0.0f;
#pragma unroll
                        for (int a2 = 0; a2 < W; ++a2) {
                            const float2 v = win[base + a2];
                            sr = fmaf(v.x, wt[2][a2], sr);
                            si = fmaf(v.y, wt[2][a2], si);
                        }
                        const float w01 = wt[0][a0] * wt[1][a1];
                        ar = fmaf(sr, w01, ar);
                        ai = fmaf(si, w01, ai);
                    }
                }
            }
            float2 r = make_float2(ar, ai);
            if (post) {
                const float2 pv = post[j];
                r = make_float2(ar * pv.x - ai * pv.y, ar * pv.y + ai * pv.x);
            }
            out[perm[j]] = r;
        }
        if (!more) break;
        __syncthreads();
        // slide: the last w - 1 z-cells of each column to its front, ...
        float2 keep[Z::NKPT];
#pragma unroll
        for (int i = 0; i < Z::NKPT; ++i) {
            const int e = tid + i * ZI_THREADS;
            if (e < Z::NKEEP) {
                const int c = e / (W - 1), q = e % (W - 1);
                keep[i] = win[c * Z::ZP + ZI_ZT + q];
            }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < Z::NKPT; ++i) {
            const int e = tid + i * ZI_THREADS;
            if (e < Z::NKEEP) {
                const int c = e / (W - 1), q = e % (W - 1);
                win[c * Z::ZP + q] = keep[i];
            }
        }
        // ... and the prefetched z-cells behind them
#pragma unroll
        for (int i = 0; i < Z::NPT; ++i) {
            const int e = tid + i * ZI_THREADS;
            if (e < Z::NNEW) {
                const int c = e / ZI_ZT, q = e % ZI_ZT;
                win[c * Z::ZP + (W - 1) + q] = nxt[i];
            }
        }
        __syncthreads();
    }
}

struct ZInterpArgs {
    const mn_bins *g;
    float beta;
    const int32_t *bstart;
    const uint32_t *perm;
    CI3s i1s;
    CF3s frs;
    const float2 *grid, *post;
    float2 *out;
    hipStream_t s;
};

constexpr int ZI_SEGBINS = 16;  // z-bins per workgroup (one slide per bin)

template <int DIM, int W>
struct ZInterpLaunch {
    static int run(const ZInterpArgs &a) {
        if constexpr (DIM != 3 || W < 2 || W > 12) {
            set_error("interp zstream: needs 3D and 2 <= w <= 12");
            return MN_EINVAL;
        } else {
            using Z = ZWin<W>;
            if (Z::LDS > (size_t)max_lds_per_block()) {
                set_error("interp zstream: window does not fit in LDS");
                return MN_EINVAL;
            }
            Geom g = make_geom(a.g);
            const float bl2e = (float)(a.beta * 1.4426950408889634);
            const float inv_hw = (float)(2.0 / W);
            const int nseg = (g.nb[2] + ZI_SEGBINS - 1) / ZI_SEGBINS;
            const int64_t nwg = (int64_t)g.nb[0] * g.nb[1] * nseg;
            auto kern = k_interp_zstream<W>;
            if (Z::LDS > 65536)
                MN_HIP_CHECK(hipFuncSetAttribute(
                    (const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)Z::LDS));
            kern<<<(unsigned)nwg, ZI_THREADS, Z::LDS, a.s>>>(g, bl2e, inv_hw, nseg, ZI_SEGBINS,
                                                             a.bstart, a.perm, a.i1s, a.frs,
                                                             a.grid, a.post, a.out);
            MN_LAUNCH_CHECK("interp zstream");
            return MN_OK;
        }
    }
};

}  // namespace

int check_points(const mn_bins *g, int64_t P, int64_t nsub, const int32_t *info,
                 const uint32_t *perm, const int32_t *const i1s[3], const float *const frs[3],
                 CI3s *ci, CF3s *cf) {
    MN_REQUIRE(P >= 1 && P < (int64_t(1) << 31), "P must be in [1, 2^31)");
    MN_REQUIRE(nsub >= 0 && nsub < (int64_t(1) << 31), "nsub out of range");
    MN_REQUIRE(nsub == 0 || (info && perm), "NULL subproblem table or permutation");
    *ci = CI3s{};
    *cf = CF3s{};
    for (int d = 0; d < g->dim; ++d) {
        MN_REQUIRE(i1s[d] && frs[d], "NULL sorted cell/fraction pointer");
        ci->p[d] = i1s[d];
        cf->p[d] = frs[d];
    }
    return MN_OK;
}

}  // namespace mn

using namespace mn;

extern "C" {

int mn_interp(const mn_bins *g, float beta, int64_t P, int64_t nsub, const int32_t *sub_info,
              const uint32_t *perm, const int32_t *const i1s[3], const float *const frs[3],
              const void *grid, const void *post, void *out, mn_stream_t stream) {
    clear_error();
    int rc = check_bins(g);
    if (rc) return rc;
    InterpArgs a{};
    rc = check_points(g, P, nsub, sub_info, perm, i1s, frs, &a.i1s, &a.frs);
    if (rc) return rc;
    MN_REQUIRE(grid && out, "interp: NULL grid or output");
    a.g = g;
    a.beta = beta;
    a.nsub = nsub;
    a.info = sub_info;
    a.perm = perm;
    a.grid = static_cast<const float2 *>(grid);
    a.post = static_cast<const float2 *>(post);
    a.out = static_cast<float2 *>(out);
    a.s = as_stream(stream);
    return select_dim_w<InterpLaunch>(g->dim, g->w, a);
}

int mn_interp_direct(const mn_bins *g, float beta, int64_t P, const uint32_t *perm,
                     const int32_t *const i1s[3], const float *const frs[3], const void *grid,
                     const void *post, void *out, mn_stream_t stream) {
    clear_error();
    int rc = check_bins(g);
    if (rc) return rc;
    MN_REQUIRE(g->dim == 3, "interp direct: 3D only");
    InterpArgs a{};
    rc = check_points(g, P, 0, nullptr, perm, i1s, frs, &a.i1s, &a.frs);
    if (rc) return rc;
    MN_REQUIRE(perm && grid && out, "interp direct: NULL pointer");
    a.g = g;
    a.beta = beta;
    a.nsub = P;
    a.perm = perm;
    a.grid = static_cast<const float2 *>(grid);
    a.post = static_cast<const float2 *>(post);
    a.out = static_cast<float2 *>(out);
    a.s = as_stream(stream);
    return select_dim_w<DirectInterpLaunch>(3, g->w, a);
}

int mn_interp_zstream(const mn_bins *g, float beta, int64_t P, const int32_t *bin_start,
                      const uint32_t *perm, const int32_t *const i1s[3],
                      const float *const frs[3], const void *grid, const void *post, void *out,
                      mn_stream_t stream) {
    clear_error();
    int rc = check_bins(g);
    if (rc) return rc;
    MN_REQUIRE(g->dim == 3 && g->m[0] == ZI_BX && g->m[1] == ZI_BY && g->m[2] == ZI_ZT,
               "interp zstream: bins must be 3D with m = (16, 16, 8)");
    ZInterpArgs a{};
    rc = check_points(g, P, 0, nullptr, perm, i1s, frs, &a.i1s, &a.frs);
    if (rc) return rc;
    MN_REQUIRE(bin_start && perm && grid && out, "interp zstream: NULL pointer");
    a.g = g;
    a.beta = beta;
    a.bstart = bin_start;
    a.perm = perm;
    a.grid = static_cast<const float2 *>(grid);
    a.post = static_cast<const float2 *>(post);
    a.out = static_cast<float2 *>(out);
    a.s = as_stream(stream);
    return select_dim_w<ZInterpLaunch>(3, g->w, a);
}

}  // extern "C"
