// Spreading (type-1 core) on LDS-staged subproblem tiles.
//
// One 256-thread workgroup per subproblem (<= msub bin-sorted points of one
// bin). The padded tile of the bin (m + w - 1 cells per dim) lives in LDS as
// two fp64 planes (re, im). Each lane takes one point at a time: it gathers
// the strength c[perm[j]] (caller order; optionally times the type-3
// prephase), evaluates the w ES weights per dim once, and adds the w^dim
// taps into LDS with ds_add_f64. On CDNA4 fp32 LDS atomics retire about one
// lane every two clocks per CU, several times slower than fp64 ones, and the
// fp64 tile also sums more accurately. After a barrier the tile is flushed
// to the periodic fine grid with global atomics (fp32, or fp64 into a
// complex128 grid), one component per lane so that an instruction's lanes
// hit adjacent addresses, skipping components that stayed zero. Workgroups
// are remapped so each XCD walks a contiguous run of bins. 3D fp64 tiles of
// at most 16 cells per dim are accumulated on the matrix cores instead
// (k_spread_tile_mfma).
// ref: nd.py:492-579 (OD spread), nd.py:683-742 (batched), gpu_t3.py:565-591.
#include "mn_common.h"

#include <cstdlib>
#include <type_traits>

namespace mn {

namespace {

struct SpreadArgs {
    const mn_bins *g;
    float beta;
    int64_t P, nsub;
    const int32_t *info;
    const uint32_t *perm;
    CI3s i1s;
    CF3s frs;
    const float2 *c;    // strengths (caller order); batched: B x P
    const float2 *pre;  // optional sorted-order multiplier
    void *grid;  // complex64, or complex128 when f64
    bool f64;    // fp64 strength x weight products and a complex128 grid
    int64_t b0;  // first vector of this launch (batched)
    int bc;      // vectors in this launch
    hipStream_t s;
};

__device__ __forceinline__ int wrap_tile(int v, int n) {
    v = wrap1(v, n);
    if (v >= n) v -= n;
    return v;
}

// Cell coordinate of point j relative to its bin's tile (in [0, m)), or -1.
__device__ __forceinline__ int local_cell(int i1, int hw, int n, int b, int m) {
    int v = wrap1(i1 + hw, n);
    if ((unsigned)v >= (unsigned)n) v = pmod(v, n);
    int loc = v - b * m;
    return ((unsigned)loc < (unsigned)m) ? loc : -1;
}

// F64: the strength times its prephase and every tap product are formed in
// fp64 and the grid is complex128 (flushed with fp64 atomics), so the grid
// carries no white fp32 rounding noise; the ES weights stay fp32, evaluated
// without the cancellation of sqrt(1 - z^2) - 1 (es_weight_stable: at eps
// 1e-6 the plain fp32 exponent alone doubled the type-3 error).
template <int DIM, int W, bool BATCH, bool F64>
__global__ __launch_bounds__(256) void k_spread_tiled(Geom g, float bl2e, float inv_hw,
                                                      int64_t nsub, const int32_t *__restrict__ info,
                                                      const uint32_t *__restrict__ perm, CI3s i1s,
                                                      CF3s frs, const float2 *__restrict__ c,
                                                      const float2 *__restrict__ pre,
                                                      void *__restrict__ grid, int64_t P,
                                                      int64_t b0, int bc) {
    using Real = typename std::conditional<F64, double, float>::type;
    extern __shared__ double lds[];
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
    const int nvec = BATCH ? bc : 1;
    for (int q = threadIdx.x; q < 2 * T * nvec; q += 256) lds[q] = 0.0;

    // 3D fp64 tiles: the lanes of one atomic instruction add the same tap
    // offset to their points' tile bases, so two lanes whose bases agree
    // modulo 32 doubles (the 64 four-byte banks) collide. The subproblem's
    // points are taken in an order that deals them round-robin over the 32
    // residues of their base (round k holds the k-th point of every residue
    // that has one), so that consecutive lanes hit distinct banks while
    // every residue still has points.
    constexpr bool RORD = F64 && DIM == 3;
    constexpr int ORD_MAX = 1024;  // points per subproblem the reordering takes
    __shared__ uint16_t ord[RORD ? ORD_MAX : 1];
    __shared__ int rcnt[32];
    const bool use_ord = RORD && cnt <= ORD_MAX;
    if (use_ord) {
        if (threadIdx.x < 32) rcnt[threadIdx.x] = 0;
        __syncthreads();
        constexpr int NI = ORD_MAX / 256;
        int res[NI], rk[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int t = threadIdx.x + 256 * i;
            res[i] = rk[i] = 0;
            if (t < cnt) {
                const int64_t j = (int64_t)s0 + t;
                int lc[3];
#pragma unroll
                for (int d = 0; d < 3; ++d)
                    lc[d] = local_cell(i1s.p[d][j], W / 2, g.n[d], b[d], g.m[d]);
                res[i] = (((lc[0] * p1 + lc[1]) * p2 + lc[2]) & 31);
                rk[i] = atomicAdd(&rcnt[res[i]], 1);
            }
        }
        __syncthreads();
        // slot = points in earlier rounds (sum over residues of min(n_r, k))
        // plus the residues below this one that reach round k
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int t = threadIdx.x + 256 * i;
            if (t < cnt) {
                int slot = 0;
#pragma unroll
                for (int r = 0; r < 32; ++r) {
                    const int n = rcnt[r];
                    slot += min(n, rk[i]) + ((r < res[i] && n > rk[i]) ? 1 : 0);
                }
                ord[slot] = (uint16_t)t;
            }
        }
    }
    __syncthreads();

    for (int t0 = threadIdx.x; t0 < cnt; t0 += 256) {
        const int t = use_ord ? (int)ord[t0] : t0;
        const int64_t j = (int64_t)s0 + t;
        const uint32_t src = perm[j];
        float wt[DIM][W];
        int loc[3] = {0, 0, 0};
        bool ok = true;
#pragma unroll
        for (int d = 0; d < DIM; ++d) {
            loc[d] = local_cell(i1s.p[d][j], W / 2, g.n[d], b[d], g.m[d]);
            ok = ok && loc[d] >= 0;
            const float f = frs.p[d][j];
#pragma unroll
            for (int a = 0; a < W; ++a)
                wt[d][a] = F64 ? es_weight_stable((float)a - f, bl2e, inv_hw)
                               : es_weight((float)a - f, bl2e, inv_hw);
        }
        if (!ok) continue;  // cannot happen for keys built by setpts
        float2 pv = make_float2(1.0f, 0.0f);
        if (!BATCH && pre) pv = pre[j];
        for (int v = 0; v < nvec; ++v) {
            const float2 c0 = BATCH ? c[(b0 + v) * P + src] : c[src];
            Real cvx = c0.x, cvy = c0.y;
            if (!BATCH && pre) {
                const Real px = pv.x, py = pv.y;
                const Real rx = cvx * px - cvy * py;
                cvy = cvx * py + cvy * px;
                cvx = rx;
            }
            double *tre = lds + (size_t)2 * T * v;
            double *tim = tre + T;
            if constexpr (DIM == 1) {
#pragma unroll
                for (int a0 = 0; a0 < W; ++a0) {
                    const int idx = loc[0] + a0;
                    atomicAdd(&tre[idx], (double)(cvx * (Real)wt[0][a0]));
                    atomicAdd(&tim[idx], (double)(cvy * (Real)wt[0][a0]));
                }
            } else if constexpr (DIM == 2) {
#pragma unroll
                for (int a0 = 0; a0 < W; ++a0) {
                    const Real r = cvx * (Real)wt[0][a0], i = cvy * (Real)wt[0][a0];
                    const int base = (loc[0] + a0) * p1 + loc[1];
#pragma unroll
                    for (int a1 = 0; a1 < W; ++a1) {
                        atomicAdd(&tre[base + a1], (double)(r * (Real)wt[1][a1]));
                        atomicAdd(&tim[base + a1], (double)(i * (Real)wt[1][a1]));
                    }
                }
            } else {
#pragma unroll
                for (int a0 = 0; a0 < W; ++a0) {
#pragma unroll
                    for (int a1 = 0; a1 < W; ++a1) {
                        const Real w01 = (Real)wt[0][a0] * (Real)wt[1][a1];
                        const Real r = cvx * w01, i = cvy * w01;
                        const int base = ((loc[0] + a0) * p1 + loc[1] + a1) * p2 + loc[2];
#pragma unroll
                        for (int a2 = 0; a2 < W; ++a2) {
                            atomicAdd(&tre[base + a2], (double)(r * (Real)wt[2][a2]));
                            atomicAdd(&tim[base + a2], (double)(i * (Real)wt[2][a2]));
                        }
                    }
                }
            }
        }
    }
    __syncthreads();

    const int o0 = b[0] * g.m[0] - W / 2;
    const int o1 = DIM >= 2 ? b[1] * g.m[1] - W / 2 : 0;
    const int o2 = DIM >= 3 ? b[2] * g.m[2] - W / 2 : 0;
    const int64_t gsz = (int64_t)g.n[0] * g.n[1] * g.n[2];
    // one component per thread: thread e adds component e % 2 (re, im) of
    // cell e / 2, so consecutive lanes hit adjacent addresses (L2 atomics
    // are paid per cache line; with re and im in one thread the lines of an
    // instruction were half used)
    for (int e = threadIdx.x; e < 2 * T; e += 256) {
        const int q = e >> 1, comp = e & 1;
        const int q2 = q % p2, r12 = q / p2;
        const int q1 = r12 % p1, q0 = r12 / p1;
        const int g0 = wrap_tile(o0 + q0, g.n[0]);
        const int g1 = DIM >= 2 ? wrap_tile(o1 + q1, g.n[1]) : 0;
        const int g2 = DIM >= 3 ? wrap_tile(o2 + q2, g.n[2]) : 0;
        const int64_t cell = ((int64_t)g0 * g.n[1] + g1) * g.n[2] + g2;
        for (int v = 0; v < nvec; ++v) {
            const double val = lds[(size_t)2 * T * v + (size_t)comp * T + q];
            if (val == 0.0) continue;
            if constexpr (F64) {
                unsafeAtomicAdd(reinterpret_cast<double *>(grid) + 2 * cell + comp, val);
            } else {
                float *dst = reinterpret_cast<float *>(
                    reinterpret_cast<float2 *>(grid) + (BATCH ? (b0 + v) * gsz : 0) + cell);
                unsafeAtomicAdd(dst + comp, (float)val);
            }
        }
    }
}

// 3D fp64 tile spread on the matrix cores (type-3 sources, complex128 grid),
// for padded tiles of at most 16 cells per dim. Instead of one LDS
// atomic per tap, the tile is accumulated by v_mfma_f64_16x16x4f64 outer
// products: for each x plane of the tile, D[y][z] += sum over 4 points k of
// A[y][k] B[k][z] with A = wx(x) wy(y) (exact in fp64: the weights are fp32)
// and B = c_k wz(z) (the strength times its prephase, fp64, as the
// LDS-atomic kernel forms it); the real and imaginary planes are two MFMAs
// sharing A. Wave w of the four owns the x planes w + 4 q, q < 4: eight
// 16x16 fp64 accumulators (4 planes, re and im) in registers.
// Per batch of 64 points the workgroup writes each point's x and y
// weight rows (zero outside the footprint; the x row permuted so that a
// wave's four planes are adjacent) and its two B rows (16 z cells, fp64),
// one role per thread; then every wave sweeps the batch in K-steps of 4
// points, skipping the MFMAs of a plane that none of the 4 points reaches
// (the subproblem is taken in x-footprint order, so neighbouring points
// share planes). After the last batch the accumulators are flushed to the
// grid with fp64 atomics, re and im of a cell from adjacent lanes, skipping
// zeros. Only the summation order differs from the LDS-atomic kernel.
// (Tiles of 32 x 16 x 16 cells with eight waves, bins of 33 - w along x,
// measured 5 % slower at cfg 5: 0.477 against 0.456 ms.)
typedef double mn_v4d __attribute__((ext_vector_type(4)));
constexpr int MN_SUB_MAX_ORDER = 1024;  // points per subproblem the x-order takes

template <int W>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void
k_spread_tile_mfma(Geom g, float bl2e, float inv_hw, int64_t nsub,
                   const int32_t *__restrict__ info, const uint32_t *__restrict__ perm, CI3s i1s,
                   CF3s frs, const float2 *__restrict__ c, const float2 *__restrict__ pre,
                   double *__restrict__ grid) {
    static_assert(W <= 16, "the footprint must fit a 16-cell tile");
    constexpr int NWV = 4;        // waves
    constexpr int NT = 64 * NWV;  // threads
    constexpr int PX = 4 * NWV;   // x planes
    constexpr int NB = NT / 4;    // points per batch (four roles each)
    __shared__ __align__(16) float xw[NB][PX];  // x cell x at (x % NWV) * 4 + x / NWV
    __shared__ __align__(16) float yw[NB][16];
    __shared__ __align__(16) double bre[NB][16], bim[NB][16];
    __shared__ uint32_t xmask[NB];  // planes reached by each point
    __shared__ uint16_t ord[MN_SUB_MAX_ORDER];
    __shared__ int xcnt[PX];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int64_t sub = xcd_remap(blockIdx.x, nsub);
    const int bin = info[3 * sub], s0 = info[3 * sub + 1], cnt = info[3 * sub + 2];
    int b[3];
    {
        int rem = bin;
#pragma unroll
        for (int d = 2; d >= 0; --d) {
            b[d] = rem % g.nb[d];
            rem /= g.nb[d];
        }
    }
    const int p0 = g.p[0], p1 = g.p[1], p2 = g.p[2];

    // order of the subproblem's points: by the x cell of their first tap (a
    // counting sort in LDS; within a cell, the atomics' order), so that a
    // K-step's 4 points reach few planes
    const bool ordered = cnt <= MN_SUB_MAX_ORDER;
    if (ordered) {
        if (tid < PX) xcnt[tid] = 0;
        __syncthreads();
        constexpr int NI = MN_SUB_MAX_ORDER / NT;
        int lx[NI], rk[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int t = tid + NT * i;
            lx[i] = 0;
            rk[i] = 0;
            if (t < cnt) {
                lx[i] = local_cell(i1s.p[0][(int64_t)s0 + t], W / 2, g.n[0], b[0], g.m[0]);
                lx[i] = lx[i] < 0 ? 0 : lx[i];
                rk[i] = atomicAdd(&xcnt[lx[i]], 1);
            }
        }
        __syncthreads();
        // ranks within a cell follow the atomic order, not the index order;
        // any order within a cell keeps the planes reached the same
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int t = tid + NT * i;
            if (t < cnt) {
                int base = 0;
                for (int x = 0; x < lx[i]; ++x) base += xcnt[x];
                ord[base + rk[i]] = (uint16_t)t;
            }
        }
    }

    mn_v4d are[4], aim[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        are[q] = mn_v4d{0.0, 0.0, 0.0, 0.0};
        aim[q] = mn_v4d{0.0, 0.0, 0.0, 0.0};
    }
    const int pt_role = tid & 3, pslot = tid >> 2;
    for (int bb = 0; bb < cnt; bb += NB) {
        const int nb = min(NB, cnt - bb);
        __syncthreads();  // the previous batch's K-steps are done with the tables
        {
            // prologue: point pslot of the batch, role pt_role (x row, y row,
            // B re row, B im row); rows of absent points stay zero
            const bool valid = pslot < nb;
            int t = bb + pslot;
            if (valid && ordered) t = ord[t];
            const int64_t j = (int64_t)s0 + (valid ? t : 0);
            const int d = pt_role < 2 ? pt_role : 2;
            int loc = local_cell(i1s.p[d][j], W / 2, g.n[d], b[d], g.m[d]);
            loc = loc < 0 ? 0 : loc;  // cannot happen for keys built by setpts
            const float fr = frs.p[d][j];
            float wt[W];
#pragma unroll
            for (int a = 0; a < W; ++a) wt[a] = es_weight_stable((float)a - fr, bl2e, inv_hw);
            // each thread zeroes its row, then writes its taps over it (its
            // own LDS accesses stay in order)
            if (pt_role == 0) {
                float *row = &xw[pslot][0];
                float4 *r4 = reinterpret_cast<float4 *>(row);
#pragma unroll
                for (int q = 0; q < PX / 4; ++q) r4[q] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (valid) {
#pragma unroll
                    for (int a = 0; a < W; ++a) {
                        const int x = loc + a;
                        row[(x % NWV) * 4 + x / NWV] = wt[a];
                    }
                }
            } else if (pt_role == 1) {
                float *row = &yw[pslot][0];
                float4 *r4 = reinterpret_cast<float4 *>(row);
#pragma unroll
                for (int q = 0; q < 4; ++q) r4[q] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (valid) {
#pragma unroll
                    for (int a = 0; a < W; ++a) row[loc + a] = wt[a];
                }
            }
            if (pt_role < 2) {
                if (pt_role == 0) xmask[pslot] = valid ? (((1u << W) - 1u) << loc) : 0u;
            } else {
                // the strength times its prephase, in fp64 (as the LDS kernel)
                double cv = 0.0;
                if (valid) {
                    const float2 c0 = c[perm[j]];
                    double cx = c0.x, cy = c0.y;
                    if (pre) {
                        const float2 pv = pre[j];
                        const double px = pv.x, py = pv.y;
                        const double rx = cx * px - cy * py;
                        cy = cx * py + cy * px;
                        cx = rx;
                    }
                    cv = pt_role == 2 ? cx : cy;
                }
                double *row = pt_role == 2 ? &bre[pslot][0] : &bim[pslot][0];
                double2 *r2 = reinterpret_cast<double2 *>(row);
#pragma unroll
                for (int q = 0; q < 8; ++q) r2[q] = make_double2(0.0, 0.0);
                if (valid) {
#pragma unroll
                    for (int a = 0; a < W; ++a) row[loc + a] = cv * (double)wt[a];
                }
            }
        }
        __syncthreads();
        // K-steps: lane (i, k) = (lane % 16, lane / 16) supplies A[y = i][k]
        // and B[k][z = i] of point 4 s + k
        const int i = lane & 15, k = lane >> 4;
        for (int s = 0; s < (nb + 3) >> 2; ++s) {
            const int pt = 4 * s + k;
            const uint32_t reach = xmask[4 * s] | xmask[4 * s + 1] | xmask[4 * s + 2] |
                                   xmask[4 * s + 3];
            const float4 xv = *reinterpret_cast<const float4 *>(&xw[pt][4 * wv]);
            const double yv = (double)yw[pt][i];
            const double br = bre[pt][i], bi = bim[pt][i];
            const float xs[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int x = wv + NWV * q;
                if (x < p0 && ((reach >> x) & 1u)) {
                    const double a = (double)xs[q] * yv;
                    are[q] = __builtin_amdgcn_mfma_f64_16x16x4f64(a, br, are[q], 0, 0, 0);
                    aim[q] = __builtin_amdgcn_mfma_f64_16x16x4f64(a, bi, aim[q], 0, 0, 0);
                }
            }
        }
    }

    // Flush. Lane l holds D[y = 4 r + l / 16][z = l % 16] in entry r (the
    // layout of v_mfma_f64_16x16x4f64's result, checked on MI355X). The
    // atomics go out in lane pairs: in half h, lane L adds component L % 2
    // (re, im) of the cell that lane 32 h + L / 2 holds, so one instruction
    // covers 32 whole cells, 512 contiguous bytes of a z-row pair. L2
    // atomics are paid per cache line: this took the flush at cfg 5 from
    // 0.46 to 0.16 ms against one lane per cell (re and im apart).
    const int o0 = b[0] * g.m[0] - W / 2;
    const int o1 = b[1] * g.m[1] - W / 2;
    const int o2 = b[2] * g.m[2] - W / 2;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int x = wv + NWV * q;
        if (x >= p0) continue;
        const int g0 = wrap_tile(o0 + x, g.n[0]);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int src = 32 * h + (lane >> 1);
                const double vre = __shfl(are[q][r], src, 64);
                const double vim = __shfl(aim[q][r], src, 64);
                const double v = (lane & 1) ? vim : vre;
                const int z = src & 15, y = 4 * r + (src >> 4);
                if (z < p2 && y < p1 && v != 0.0) {
                    const int g1 = wrap_tile(o1 + y, g.n[1]);
                    const int g2 = wrap_tile(o2 + z, g.n[2]);
                    unsafeAtomicAdd(grid + 2 * (((int64_t)g0 * g.n[1] + g1) * g.n[2] + g2) +
                                        (lane & 1),
                                    v);
                }
            }
        }
    }
}

// Owner-computes spread into a complex128 grid (3D): one workgroup per bin
// sums, in an fp64 LDS tile of just that bin's cells, every tap that lands
// in the bin from the points of the bins whose footprints can reach it, then
// stores the tile with plain writes. Each grid cell is written by exactly
// one workgroup, so there is no zero fill and there are no global atomics;
// a point is read by every owner its footprint may reach (about
// (1 + (w-1)/m)^3 of them), which costs little when points are sparse
// relative to the grid (type-3 grids). The reaching bins per dim are those
// whose cells meet the cyclic interval [lo - (w-1-w/2), lo + cnt - 1 + w/2]
// of point centres (centre = first tap + w/2, the sort key's cell); at most
// four per dim, found by walking that interval. Per point and dim, the taps
// inside the owner's cells come from (first tap + a - lo) mod n < cnt.
constexpr int OWN_THREADS = 256;
constexpr int OWN_MAXQ = 4;  // reaching bins per dim

// The point ranges that can reach owner bin (lo, cnt), for lane `lane` of
// the wave that calls it: every lane finds the reaching bins of each dim (a
// little arithmetic), then lane r takes combination r of them: its start in
// the sorted points (st[r]) and, by a wave scan of the range sizes, the
// number of reaching points before it (pf[r]; pf[64] = all of them).
template <int W>
__device__ __forceinline__ void owner_ranges(const Geom &g, const int (&lo)[3],
                                             const int (&cnt)[3],
                                             const int32_t *__restrict__ bstart, int tid,
                                             int *pf, int *st) {
    int qs[3][OWN_MAXQ], nq[3];
#pragma unroll
    for (int d = 0; d < 3; ++d) {
        const int n = g.n[d], m = g.m[d];
        const int len = cnt[d] + W - 1;
        nq[d] = 0;
        if (len >= n) {
            for (int q = 0; q < g.nb[d] && q < OWN_MAXQ; ++q) qs[d][nq[d]++] = q;
        } else {
            int cell = pmod(lo[d] - (W - 1 - W / 2), n), left = len;
            while (left > 0 && nq[d] < OWN_MAXQ) {
                const int q = cell / m;
                bool dup = false;
                for (int k = 0; k < nq[d]; ++k) dup = dup || qs[d][k] == q;
                if (!dup) qs[d][nq[d]++] = q;
                const int end = min(q * m + m, n);
                left -= end - cell;
                cell = end == n ? 0 : end;
            }
        }
    }
    const int ncomb = nq[0] * nq[1] * nq[2];
    int s0 = 0, len = 0;
    if (tid < ncomb) {
        const int i2 = tid % nq[2], i01 = tid / nq[2];
        const int i1 = i01 % nq[1], i0 = i01 / nq[1];
        const int64_t nbr = ((int64_t)qs[0][i0] * g.nb[1] + qs[1][i1]) * g.nb[2] + qs[2][i2];
        s0 = bstart[nbr];
        len = bstart[nbr + 1] - s0;
    }
    int incl = len;
#pragma unroll
    for (int k = 1; k < 64; k <<= 1) {
        const int v = __shfl_up(incl, k, 64);
        incl += tid >= k ? v : 0;
    }
    pf[tid] = incl - len;
    st[tid] = s0;
    if (tid == 63) pf[64] = incl;
}

template <int W>
__global__ __launch_bounds__(OWN_THREADS) void k_spread_owner(
    Geom g, float bl2e, float inv_hw, int64_t nbins, const int32_t *__restrict__ bstart,
    const uint32_t *__restrict__ perm, CI3s i1s, CF3s frs, const float2 *__restrict__ c,
    const float2 *__restrict__ pre, double2 *__restrict__ grid) {
    extern __shared__ double own[];
    __shared__ int pf[OWN_MAXQ * OWN_MAXQ * OWN_MAXQ + 1];
    __shared__ int st[OWN_MAXQ * OWN_MAXQ * OWN_MAXQ];
    const int tid = threadIdx.x;
    const int64_t bin = xcd_remap(blockIdx.x, nbins);
    int b[3], lo[3], cnt[3];
    {
        int64_t rem = bin;
#pragma unroll
        for (int d = 2; d >= 0; --d) {
            b[d] = (int)(rem % g.nb[d]);
            rem /= g.nb[d];
        }
    }
#pragma unroll
    for (int d = 0; d < 3; ++d) {
        lo[d] = b[d] * g.m[d];
        cnt[d] = min(g.m[d], g.n[d] - lo[d]);
    }
    const int T = cnt[0] * cnt[1] * cnt[2];
    double *tre = own, *tim = own + T;
    if (tid < 64) owner_ranges<W>(g, lo, cnt, bstart, tid, pf, st);
    __syncthreads();
    const int tot = pf[OWN_MAXQ * OWN_MAXQ * OWN_MAXQ];
    if (tot == 0) {  // no point reaches the bin: zeros straight to the grid
        const int PL = cnt[1] * cnt[2];
        const int64_t n12 = (int64_t)g.n[1] * g.n[2];
        for (int t = tid; t < PL; t += OWN_THREADS) {
            const int e1 = t / cnt[2], e2 = t - e1 * cnt[2];
            double2 *dst =
                grid + (int64_t)lo[0] * n12 + (int64_t)(lo[1] + e1) * g.n[2] + lo[2] + e2;
            for (int e0 = 0; e0 < cnt[0]; ++e0) dst[(int64_t)e0 * n12] = make_double2(0.0, 0.0);
        }
        return;
    }
    for (int i = tid; i < 2 * T; i += OWN_THREADS) own[i] = 0.0;
    __syncthreads();
    int q = 0;
    for (int t = tid; t < tot; t += OWN_THREADS) {
        while (t >= pf[q + 1]) ++q;
        const int64_t j = (int64_t)st[q] + (t - pf[q]);
        // owner-local cell of each tap per dim (>= cnt: outside the bin);
        // dims 1 and 2 as register arrays, dim 0 inline in the outer loop
        int a00 = pmod(lo[0] - i1s.p[0][j], g.n[0]);
        bool any = a00 < W || a00 > g.n[0] - cnt[0];
        int loc[2][W];
#pragma unroll
        for (int d = 1; d < 3; ++d) {
            const int n = g.n[d];
            const int a0 = pmod(lo[d] - i1s.p[d][j], n);
            bool hit = false;
#pragma unroll
            for (int a = 0; a < W; ++a) {
                int v = a - a0;
                v += v < 0 ? n : 0;
                loc[d - 1][a] = v;
                hit = hit || v < cnt[d];
            }
            any = any && hit;
        }
        if (!any) continue;
        float wt[2][W];
#pragma unroll
        for (int d = 1; d < 3; ++d) {
            const float f = frs.p[d][j];
#pragma unroll
            for (int a = 0; a < W; ++a)
                wt[d - 1][a] =
                    loc[d - 1][a] < cnt[d] ? es_weight_stable((float)a - f, bl2e, inv_hw) : 0.0f;
        }
        const float f0 = frs.p[0][j];
        const float2 c0 = c[perm[j]];
        double cvx = c0.x, cvy = c0.y;
        if (pre) {
            const float2 pv = pre[j];
            const double px = pv.x, py = pv.y;
            const double rx = cvx * px - cvy * py;
            cvy = cvx * py + cvy * px;
            cvx = rx;
        }
        for (int a0 = 0; a0 < W; ++a0) {
            int v0 = a0 - a00;
            v0 += v0 < 0 ? g.n[0] : 0;
            if (v0 >= cnt[0]) continue;
            const double w0 = (double)es_weight_stable((float)a0 - f0, bl2e, inv_hw);
            const double r0 = cvx * w0, i0 = cvy * w0;
#pragma unroll
            for (int a1 = 0; a1 < W; ++a1) {
                if (loc[0][a1] >= cnt[1]) continue;
                const double r = r0 * (double)wt[0][a1], im = i0 * (double)wt[0][a1];
                const int base = (v0 * cnt[1] + loc[0][a1]) * cnt[2];
#pragma unroll
                for (int a2 = 0; a2 < W; ++a2) {
                    if (loc[1][a2] >= cnt[2]) continue;
                    atomicAdd(&tre[base + loc[1][a2]], r * (double)wt[1][a2]);
                    atomicAdd(&tim[base + loc[1][a2]], im * (double)wt[1][a2]);
                }
            }
        }
    }
    __syncthreads();
    // store: thread t owns cell (e1, e2) of every x-plane of the bin, so the
    // index arithmetic is done once and each plane is written row by row
    const int PL = cnt[1] * cnt[2];
    const int64_t n12 = (int64_t)g.n[1] * g.n[2];
    for (int t = tid; t < PL; t += OWN_THREADS) {
        const int e1 = t / cnt[2], e2 = t - e1 * cnt[2];
        double2 *dst = grid + (int64_t)lo[0] * n12 + (int64_t)(lo[1] + e1) * g.n[2] + lo[2] + e2;
        for (int e0 = 0; e0 < cnt[0]; ++e0)
            dst[(int64_t)e0 * n12] = make_double2(tre[e0 * PL + t], tim[e0 * PL + t]);
    }
}

// Owner-computes spread on the matrix cores, for owner bins of at most 16
// cells per dim: the bin is accumulated like a k_spread_tile_mfma tile (a
// wave per four x planes, v_mfma_f64_16x16x4f64 outer products of the x-y
// weight products with the strength-weighted z rows, planes that none of a
// K-step's points reaches skipped), from the points of every reaching bin
// whose footprint meets the bin (compacted per chunk of reaching points, in
// order of the first x cell they reach), each tap kept only when it lands
// inside the bin. The bin is then stored with plain writes, zeros included,
// so that every cell is written by one workgroup.
template <int W>
__global__ __launch_bounds__(OWN_THREADS) __attribute__((amdgpu_waves_per_eu(3))) void
k_spread_owner_mfma(Geom g, float bl2e, float inv_hw, int64_t nbins,
                    const int32_t *__restrict__ bstart, const uint32_t *__restrict__ perm,
                    CI3s i1s, CF3s frs, const float2 *__restrict__ c,
                    const float2 *__restrict__ pre, double2 *__restrict__ grid) {
    static_assert(OWN_THREADS == 256, "four waves");
    constexpr int NB = 64;  // points per batch (four roles each)
    __shared__ __align__(16) float xw[NB][16];  // x cell x at (x & 3) * 4 + (x >> 2)
    __shared__ __align__(16) float yw[NB][16];
    __shared__ __align__(16) double bre[NB][16], bim[NB][16];
    __shared__ uint32_t xmask[NB];
    __shared__ int32_t ordj[MN_SUB_MAX_ORDER];  // sorted index of each ordered point
    __shared__ int xcnt[16];
    __shared__ int pf[OWN_MAXQ * OWN_MAXQ * OWN_MAXQ + 1];
    __shared__ int st[OWN_MAXQ * OWN_MAXQ * OWN_MAXQ];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int64_t bin = xcd_remap(blockIdx.x, nbins);
    int b[3], lo[3], cnt[3];
    {
        int64_t rem = bin;
#pragma unroll
        for (int d = 2; d >= 0; --d) {
            b[d] = (int)(rem % g.nb[d]);
            rem /= g.nb[d];
        }
    }
#pragma unroll
    for (int d = 0; d < 3; ++d) {
        lo[d] = b[d] * g.m[d];
        cnt[d] = min(g.m[d], g.n[d] - lo[d]);
    }
    if (tid < 64) owner_ranges<W>(g, lo, cnt, bstart, tid, pf, st);
    __syncthreads();
    const int tot = pf[OWN_MAXQ * OWN_MAXQ * OWN_MAXQ];
    // sorted index of reaching point t: its range q (pf[q] <= t < pf[q + 1],
    // a binary search) and its place in that range
    auto point = [&](int t) __attribute__((always_inline)) {
        int qa = 0, qb = OWN_MAXQ * OWN_MAXQ * OWN_MAXQ;
        while (qb - qa > 1) {
            const int mid = (qa + qb) >> 1;
            if (pf[mid] <= t) qa = mid;
            else qb = mid;
        }
        return st[qa] + (t - pf[qa]);
    };
    // whether the footprint of a point whose first tap along d is i1 meets
    // the bin along d, and its first in-bin cell (taps land at
    // (i1 + a - lo) mod n; a footprint entering from below starts at 0)
    auto meets = [&](int i1, int d) __attribute__((always_inline)) {
        const int v = pmod(i1 - lo[d], g.n[d]);
        return v < cnt[d] || v + W - 1 >= g.n[d];
    };
    auto first_x = [&](int i1) __attribute__((always_inline)) {
        const int v = pmod(i1 - lo[0], g.n[0]);
        return v < cnt[0] ? v : 0;
    };

    mn_v4d are[4], aim[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        are[q] = mn_v4d{0.0, 0.0, 0.0, 0.0};
        aim[q] = mn_v4d{0.0, 0.0, 0.0, 0.0};
    }
    const int pt_role = tid & 3, pslot = tid >> 2;
    // Chunks of up to MN_SUB_MAX_ORDER reaching points: most of a reaching
    // bin's points do not touch this bin, so each chunk is first compacted
    // to the points whose footprint meets the bin in all three dims, in
    // order of their first x cell (a counting sort in LDS)
    for (int c0 = 0; c0 < tot; c0 += MN_SUB_MAX_ORDER) {
        const int cn = min(MN_SUB_MAX_ORDER, tot - c0);
        __syncthreads();  // the previous chunk's batches are done with ordj
        if (tid < 16) xcnt[tid] = 0;
        __syncthreads();
        constexpr int NI = MN_SUB_MAX_ORDER / OWN_THREADS;
        // in steps over the thread's NI candidates, so that each step's
        // loads are in flight together: the sorted indices, the x cells,
        // then the y and z cells of the candidates that meet the bin in x
        int lx[NI], rk[NI], jj[NI], cx[NI], cy[NI], cz[NI];
        bool mx[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int t = tid + OWN_THREADS * i;
            jj[i] = t < cn ? point(c0 + t) : 0;
        }
#pragma unroll
        for (int i = 0; i < NI; ++i) cx[i] = i1s.p[0][jj[i]];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            mx[i] = tid + OWN_THREADS * i < cn && meets(cx[i], 0);
            cy[i] = mx[i] ? i1s.p[1][jj[i]] : 0;
            cz[i] = mx[i] ? i1s.p[2][jj[i]] : 0;
        }
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            lx[i] = -1;
            rk[i] = 0;
            if (mx[i] && meets(cy[i], 1) && meets(cz[i], 2)) {
                lx[i] = first_x(cx[i]);
                rk[i] = atomicAdd(&xcnt[lx[i]], 1);
            }
        }
        __syncthreads();
        int nkeep = 0;
#pragma unroll
        for (int x = 0; x < 16; ++x) nkeep += xcnt[x];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            if (lx[i] >= 0) {
                int base = 0;
                for (int x = 0; x < lx[i]; ++x) base += xcnt[x];
                ordj[base + rk[i]] = jj[i];
            }
        }
        for (int bb = 0; bb < nkeep; bb += NB) {
            const int nb = min(NB, nkeep - bb);
            __syncthreads();  // ordj is written; the previous K-steps are done
            {
                const bool valid = pslot < nb;
                const int64_t j = valid ? ordj[bb + pslot] : 0;
                const int d = pt_role < 2 ? pt_role : 2;
                const int n = g.n[d];
                // tap a lands at in-bin cell (a - a0) mod n; kept when below cnt
                const int a0 = pmod(lo[d] - i1s.p[d][j], n);
                const float fr = frs.p[d][j];
                int v[W];
                float wt[W];
#pragma unroll
                for (int a = 0; a < W; ++a) {
                    int va = a - a0;
                    va += va < 0 ? n : 0;
                    v[a] = va;
                    wt[a] = es_weight_stable((float)a - fr, bl2e, inv_hw);
                }
                if (pt_role == 0) {
                    float *row = &xw[pslot][0];
                    float4 *r4 = reinterpret_cast<float4 *>(row);
#pragma unroll
                    for (int q = 0; q < 4; ++q) r4[q] = make_float4(0.f, 0.f, 0.f, 0.f);
                    uint32_t mask = 0;
                    if (valid) {
#pragma unroll
                        for (int a = 0; a < W; ++a)
                            if (v[a] < cnt[0]) {
                                row[(v[a] & 3) * 4 + (v[a] >> 2)] = wt[a];
                                mask |= 1u << v[a];
                            }
                    }
                    xmask[pslot] = mask;
                } else if (pt_role == 1) {
                    float *row = &yw[pslot][0];
                    float4 *r4 = reinterpret_cast<float4 *>(row);
#pragma unroll
                    for (int q = 0; q < 4; ++q) r4[q] = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (valid) {
#pragma unroll
                        for (int a = 0; a < W; ++a)
                            if (v[a] < cnt[1]) row[v[a]] = wt[a];
                    }
                } else {
                    double cv = 0.0;
                    if (valid) {
                        const float2 c0v = c[perm[j]];
                        double cx = c0v.x, cy = c0v.y;
                        if (pre) {
                            const float2 pv = pre[j];
                            const double px = pv.x, py = pv.y;
                            const double rx = cx * px - cy * py;
                            cy = cx * py + cy * px;
                            cx = rx;
                        }
                        cv = pt_role == 2 ? cx : cy;
                    }
                    double *row = pt_role == 2 ? &bre[pslot][0] : &bim[pslot][0];
                    double2 *r2 = reinterpret_cast<double2 *>(row);
#pragma unroll
                    for (int q = 0; q < 8; ++q) r2[q] = make_double2(0.0, 0.0);
                    if (valid) {
#pragma unroll
                        for (int a = 0; a < W; ++a)
                            if (v[a] < cnt[2]) row[v[a]] = cv * (double)wt[a];
                    }
                }
            }
            __syncthreads();
            const int i = lane & 15, k = lane >> 4;
            for (int s = 0; s < (nb + 3) >> 2; ++s) {
                const int pt = 4 * s + k;
                const uint32_t reach = xmask[4 * s] | xmask[4 * s + 1] | xmask[4 * s + 2] |
                                       xmask[4 * s + 3];
                const float4 xv = *reinterpret_cast<const float4 *>(&xw[pt][4 * wv]);
                const double yv = (double)yw[pt][i];
                const double br = bre[pt][i], bi = bim[pt][i];
                const float xs[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int x = wv + 4 * q;
                    if (x < cnt[0] && ((reach >> x) & 1u)) {
                        const double a = (double)xs[q] * yv;
                        are[q] = __builtin_amdgcn_mfma_f64_16x16x4f64(a, br, are[q], 0, 0, 0);
                        aim[q] = __builtin_amdgcn_mfma_f64_16x16x4f64(a, bi, aim[q], 0, 0, 0);
                    }
                }
            }
        }
    }

    // store: lane l holds D[y = 4 r + l / 16][z = l % 16] in entry r; 16
    // lanes write one 256-byte z-row
    const int64_t n12 = (int64_t)g.n[1] * g.n[2];
    const int z = lane & 15;
    if (z >= cnt[2]) return;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int x = wv + 4 * q;
        if (x >= cnt[0]) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int y = 4 * r + (lane >> 4);
            if (y >= cnt[1]) continue;
            grid[(int64_t)(lo[0] + x) * n12 + (int64_t)(lo[1] + y) * g.n[2] + lo[2] + z] =
                make_double2(are[q][r], aim[q][r]);
        }
    }
}

struct OwnerArgs {
    const mn_bins *g;
    float beta;
    const int32_t *bstart;
    const uint32_t *perm;
    CI3s i1s;
    CF3s frs;
    const float2 *c, *pre;
    double2 *grid;
    hipStream_t s;
};

// Owner bins of at most 16 cells per dim go through the matrix cores unless
// MN_T3_OWNER_MFMA=0 (read at every launch).
inline bool spread_owner_mfma() {
    const char *e = std::getenv("MN_T3_OWNER_MFMA");
    return !(e && std::atoi(e) == 0);
}

template <int DIM, int W>
struct OwnerLaunch {
    static int run(const OwnerArgs &a) {
        if constexpr (DIM != 3) {
            set_error("spread_owner: 3D only");
            return MN_EINVAL;
        } else {
            Geom g = make_geom(a.g);
            const size_t lds = (size_t)16 * g.m[0] * g.m[1] * g.m[2];
            if (lds > (size_t)max_lds_per_block()) {
                set_error("spread_owner: bin does not fit in LDS; use smaller bins");
                return MN_EINVAL;
            }
            const int64_t nb = nbins_total(a.g);
            const float bl2e = (float)(a.beta * 1.4426950408889634);
            const float inv_hw = (float)(2.0 / W);
            for (int d = 0; d < 3; ++d)
                if (g.nb[d] > 1 && g.m[d] < W - 1) {
                    set_error("spread_owner: bins must be at least w - 1 cells wide");
                    return MN_EINVAL;
                }
            // (a footprint longer than an axis would land twice on a cell)
            if (g.m[0] <= 16 && g.m[1] <= 16 && g.m[2] <= 16 && g.n[0] >= W && g.n[1] >= W &&
                g.n[2] >= W && spread_owner_mfma()) {
                k_spread_owner_mfma<W><<<(unsigned)nb, OWN_THREADS, 0, a.s>>>(
                    g, bl2e, inv_hw, nb, a.bstart, a.perm, a.i1s, a.frs, a.c, a.pre, a.grid);
                MN_LAUNCH_CHECK("spread_owner (matrix cores)");
                return MN_OK;
            }
            auto kern = k_spread_owner<W>;
            if (lds > 60000)  // with the static range tables, past the 64 KB default
                MN_HIP_CHECK(hipFuncSetAttribute(
                    (const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
            kern<<<(unsigned)nb, OWN_THREADS, lds, a.s>>>(g, bl2e, inv_hw, nb, a.bstart, a.perm,
                                                          a.i1s, a.frs, a.c, a.pre, a.grid);
            MN_LAUNCH_CHECK("spread_owner");
            return MN_OK;
        }
    }
};

// The fp64 3D tiles go through the matrix cores unless MN_T3_TILE_MFMA=0
// (read at every launch, so that a test can compare both kernels).
inline bool spread_tile_mfma() {
    const char *e = std::getenv("MN_T3_TILE_MFMA");
    return !(e && std::atoi(e) == 0);
}

template <int DIM, int W>
struct SpreadLaunch {
    static int run(const SpreadArgs &a) {
        Geom g = make_geom(a.g);
        const float bl2e = (float)(a.beta * 1.4426950408889634);
        const float inv_hw = (float)(2.0 / W);
        const int64_t T = tile_cells(a.g);
        const bool batch = a.bc > 1 || a.b0 > 0;
        const size_t lds = (size_t)2 * T * sizeof(double) * (batch ? a.bc : 1);
        if (lds > (size_t)max_lds_per_block()) {
            set_error("spread: tile does not fit in LDS; use smaller bins");
            return MN_EINVAL;
        }
        if (a.nsub == 0) return MN_OK;
        if constexpr (DIM == 3 && W <= 16) {
            if (a.f64 && !batch && g.p[0] <= 16 && g.p[1] <= 16 && g.p[2] <= 16 &&
                spread_tile_mfma()) {
                k_spread_tile_mfma<W><<<(unsigned)a.nsub, 256, 0, a.s>>>(
                    g, bl2e, inv_hw, a.nsub, a.info, a.perm, a.i1s, a.frs, a.c, a.pre,
                    static_cast<double *>(a.grid));
                MN_LAUNCH_CHECK("spread (matrix-core tiles)");
                return MN_OK;
            }
        }
        auto kern = batch   ? k_spread_tiled<DIM, W, true, false>
                    : a.f64 ? k_spread_tiled<DIM, W, false, true>
                            : k_spread_tiled<DIM, W, false, false>;
        if (lds > 65536)
            MN_HIP_CHECK(hipFuncSetAttribute((const void *)kern,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        kern<<<(unsigned)a.nsub, 256, lds, a.s>>>(g, bl2e, inv_hw, a.nsub, a.info, a.perm, a.i1s,
                                                  a.frs, a.c, a.pre, a.grid, a.P, a.b0, a.bc);
        MN_LAUNCH_CHECK("spread");
        return MN_OK;
    }
};

}  // namespace

}  // namespace mn

using namespace mn;


static int spread_impl(const mn_bins *g, float beta, int64_t P, int64_t nsub,
                       const int32_t *sub_info, const uint32_t *perm,
                       const int32_t *const i1s[3], const float *const frs[3], const void *c,
                       const void *pre, void *grid, bool zero, bool f64, mn_stream_t stream) {
    clear_error();
    int rc = check_bins(g);
    if (rc) return rc;
    SpreadArgs a{};
    rc = check_points(g, P, nsub, sub_info, perm, i1s, frs, &a.i1s, &a.frs);
    if (rc) return rc;
    MN_REQUIRE(c && grid, "spread: NULL strengths or grid");
    int64_t gsz = 1;
    for (int d = 0; d < g->dim; ++d) gsz *= g->n[d];
    a.g = g;
    a.beta = beta;
    a.P = P;
    a.nsub = nsub;
    a.info = sub_info;
    a.perm = perm;
    a.c = static_cast<const float2 *>(c);
    a.pre = static_cast<const float2 *>(pre);
    a.grid = grid;
    a.f64 = f64;
    a.b0 = 0;
    a.bc = 1;
    a.s = as_stream(stream);
    if (zero) {
        rc = fill_zero(grid, gsz * (f64 ? 16 : 8), a.s);
        if (rc) return rc;
    }
    return select_dim_w<SpreadLaunch>(g->dim, g->w, a);
}

extern "C" {

int mn_spread(const mn_bins *g, float beta, int64_t P, int64_t nsub, const int32_t *sub_info,
              const uint32_t *perm, const int32_t *const i1s[3], const float *const frs[3],
              const void *c, const void *pre, void *grid, mn_stream_t stream) {
    return spread_impl(g, beta, P, nsub, sub_info, perm, i1s, frs, c, pre, grid, true, false,
                       stream);
}

int mn_spread_c128(const mn_bins *g, float beta, int64_t P, int64_t nsub,
                   const int32_t *sub_info, const uint32_t *perm, const int32_t *const i1s[3],
                   const float *const frs[3], const void *c, const void *pre, void *grid,
                   mn_stream_t stream) {
    return spread_impl(g, beta, P, nsub, sub_info, perm, i1s, frs, c, pre, grid, true, true,
                       stream);
}

int mn_spread_owner_c128(const mn_bins *g, float beta, int64_t P, const int32_t *bin_start,
                         const uint32_t *perm, const int32_t *const i1s[3],
                         const float *const frs[3], const void *c, const void *pre, void *grid,
                         mn_stream_t stream) {
    clear_error();
    int rc = check_bins(g);
    if (rc) return rc;
    MN_REQUIRE(g->dim == 3, "spread_owner: 3D only");
    MN_REQUIRE(P >= 1 && P < (int64_t(1) << 31), "P must be in [1, 2^31)");
    MN_REQUIRE(bin_start && perm && c && grid, "spread_owner: NULL pointer");
    OwnerArgs a{};
    for (int d = 0; d < 3; ++d) {
        MN_REQUIRE(i1s[d] && frs[d], "NULL sorted cell/fraction pointer");
        a.i1s.p[d] = i1s[d];
        a.frs.p[d] = frs[d];
    }
    a.g = g;
    a.beta = beta;
    a.bstart = bin_start;
    a.perm = perm;
    a.c = static_cast<const float2 *>(c);
    a.pre = static_cast<const float2 *>(pre);
    a.grid = static_cast<double2 *>(grid);
    a.s = as_stream(stream);
    return select_dim_w<OwnerLaunch>(3, g->w, a);
}

int mn_spread_accumulate(const mn_bins *g, float beta, int64_t P, int64_t nsub,
                         const int32_t *sub_info, const uint32_t *perm,
                         const int32_t *const i1s[3], const float *const frs[3], const void *c,
                         const void *pre, void *grid, mn_stream_t stream) {
    return spread_impl(g, beta, P, nsub, sub_info, perm, i1s, frs, c, pre, grid, false, false,
                       stream);
}

int mn_spread_batch(const mn_bins *g, float beta, int64_t P, int64_t nsub,
                    const int32_t *sub_info, const uint32_t *perm, const int32_t *const i1s[3],
                    const float *const frs[3], int64_t B, const void *cs, void *grids,
                    mn_stream_t stream) {
    clear_error();
    int rc = check_bins(g);
    if (rc) return rc;
    SpreadArgs a{};
    rc = check_points(g, P, nsub, sub_info, perm, i1s, frs, &a.i1s, &a.frs);
    if (rc) return rc;
    MN_REQUIRE(B >= 1, "spread_batch: B must be >= 1");
    MN_REQUIRE(cs && grids, "spread_batch: NULL strengths or grids");
    int64_t gsz = 1;
    for (int d = 0; d < g->dim; ++d) gsz *= g->n[d];
    a.g = g;
    a.beta = beta;
    a.P = P;
    a.nsub = nsub;
    a.info = sub_info;
    a.perm = perm;
    a.c = static_cast<const float2 *>(cs);
    a.pre = nullptr;
    a.grid = grids;
    a.f64 = false;
    a.s = as_stream(stream);
    rc = fill_zero(grids, B * gsz * 8, a.s);
    if (rc) return rc;
    // Vectors per launch: as many fp64 tiles as fit in half of the LDS
    // (two workgroups per CU), at least one.
    const int64_t tile_bytes = 16 * tile_cells(g);
    int64_t per = (max_lds_per_block() / 2) / tile_bytes;
    if (per < 1) per = 1;
    if (per > B) per = B;
    for (int64_t v0 = 0; v0 < B; v0 += per) {
        a.b0 = v0;
        a.bc = (int)((B - v0 < per) ? (B - v0) : per);
        rc = select_dim_w<SpreadLaunch>(g->dim, g->w, a);
        if (rc) return rc;
    }
    return MN_OK;
}

}  // extern "C"
