// Plan-time point setup on the GPU in native fp64 (CDNA4 runs fp64 at half
// the fp32 vector rate, so the fold/rescale needs no double-single tricks):
//   * type 1/2: fold mod 2pi, rescale to fine-grid units, cell index + frac,
//     bin key (ref: nd.py:152-165, nd.py:308-313);
//   * type 3: source rescale + prephase, target rescale + postphase/deconv
//     (ref: gpu_t3.py:357-377, gpu_t3.py:474-488);
//   * gather of per-point arrays into sorted order.
// Floating-point contraction is disabled in this file: the fp64 sequences
// reproduce numpy's separately-rounded operations bit for bit.
#pragma clang fp contract(off)

#include "mn_common.h"

namespace mn {
namespace {

struct D3 { const double *p[3]; };
struct I3 { int32_t *p[3]; };
struct F3 { float *p[3]; };
struct CI3 { const int32_t *p[3]; };
struct CF3 { const float *p[3]; };

// np.mod(x, 2pi) for float64: fmod, then move a negative remainder up by
// 2pi; a zero remainder becomes +0.
__device__ __forceinline__ double np_mod_2pi(double x) {
    double r = fmod(x, kTwoPi);
    if (r != 0.0) {
        if (r < 0.0) r += kTwoPi;
    } else {
        r = 0.0;
    }
    return r;
}

// Bin coordinate of a cell index along one dim (see mn_bins).
__device__ __forceinline__ int bin_of(int i1, int hw, int n, int m) {
    int v = i1 + hw;
    v = wrap1(v, n);
    if ((unsigned)v >= (unsigned)n) v = pmod(v, n);
    return v / m;
}

// Cell index and fraction of one coordinate along one dim (crit64 when
// prec64, else the fp32 path); see mn_setpts_t12.
__device__ __forceinline__ void cell_t12(double x, double h, double halfw, int prec64, int &ii,
                                         float &f) {
    double r = np_mod_2pi(x);
    if (prec64) {
        double xi = r / h;
        ii = (int)ceil(xi - halfw);
        f = (float)(xi - (double)ii);
    } else {
        float xi = (float)r / (float)h;
        ii = (int)ceilf(xi - (float)halfw);
        f = xi - (float)ii;
    }
}

template <int DIM>
__global__ void k_setpts_t12(int64_t P, D3 x, Geom g, double h0, double h1, double h2,
                             int prec64, I3 i1o, F3 fro, uint32_t *__restrict__ key) {
    int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= P) return;
    const double hh[3] = {h0, h1, h2};
    const double halfw = 0.5 * (double)g.w;  // w/2, exact
    uint32_t k = 0;
#pragma unroll
    for (int d = 0; d < DIM; ++d) {
        int ii;
        float f;
        cell_t12(x.p[d][j], hh[d], halfw, prec64, ii, f);
        i1o.p[d][j] = ii;
        fro.p[d][j] = f;
        k = k * (uint32_t)g.nb[d] + (uint32_t)bin_of(ii, g.w / 2, g.n[d], g.m[d]);
    }
    key[j] = k;
}

// 3D setup for the z-sweep spread (GATHER false) and the z-gather
// interpolation (GATHER true): the same cells and fractions, and the packed
// point word (zs_word, zg_word) instead of a bin key.
// A thread takes ZP_ITEMS points ZP_THREADS apart (coalesced), their
// coordinate loads all issued before the arithmetic: with one point per
// thread the kernel waited on memory latency.
constexpr int ZP_THREADS = 256;
constexpr int ZP_ITEMS = 4;
template <bool GATHER>
__global__ __launch_bounds__(ZP_THREADS) void k_zs_setpts(int64_t P, D3 x, int n0, int n1, int n2,
                                                          int w, double h0, double h1, double h2,
                                                          int prec64, uint32_t *__restrict__ word,
                                                          F3 fro) {
    const int64_t j0 = (int64_t)blockIdx.x * (ZP_THREADS * ZP_ITEMS) + threadIdx.x;
    const double halfw = 0.5 * (double)w;
    const int nzc = (n2 + kZsChunk - 1) / kZsChunk;
    double xv[ZP_ITEMS][3];
#pragma unroll
    for (int i = 0; i < ZP_ITEMS; ++i) {
        const int64_t j = j0 + (int64_t)i * ZP_THREADS;
#pragma unroll
        for (int d = 0; d < 3; ++d) xv[i][d] = j < P ? x.p[d][j] : 0.0;
    }
#pragma unroll
    for (int i = 0; i < ZP_ITEMS; ++i) {
        const int64_t j = j0 + (int64_t)i * ZP_THREADS;
        if (j >= P) break;
        int ix, iy, iz;
        float fx, fy, fz;
        cell_t12(xv[i][0], h0, halfw, prec64, ix, fx);
        cell_t12(xv[i][1], h1, halfw, prec64, iy, fy);
        cell_t12(xv[i][2], h2, halfw, prec64, iz, fz);
        if constexpr (GATHER)
            word[j] = zg_word(pmod(ix, n0), pmod(iy, n1), pmod(iz, n2), n1, nzc);
        else
            word[j] = zs_word(pmod(ix, n0), pmod(iy, n1), pmod(iz, n2), n1, nzc, w);
        fro.p[0][j] = fx;
        fro.p[1][j] = fy;
        fro.p[2][j] = fz;
    }
}

// 2D type-1 setup for the y-sweep spread: the same cells and fractions, and
// the packed point word (ys_word).
__global__ void k_ys_setpts(int64_t P, D3 x, int n0, int n1, int w, double h0, double h1,
                            int prec64, uint32_t *__restrict__ word, F3 fro) {
    int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= P) return;
    const double halfw = 0.5 * (double)w;
    int ix, iy;
    float fx, fy;
    cell_t12(x.p[0][j], h0, halfw, prec64, ix, fx);
    cell_t12(x.p[1][j], h1, halfw, prec64, iy, fy);
    word[j] = ys_word(pmod(ix, n0), pmod(iy, n1), n1, w);
    fro.p[0][j] = fx;
    fro.p[1][j] = fy;
}

// 2D setup for the y-window MFMA sweep: the same cells and fractions, and
// the packed point word (ym_word).
__global__ void k_ym_setpts(int64_t P, D3 x, int n0, int n1, int w, double h0, double h1,
                            int prec64, uint32_t *__restrict__ word, F3 fro) {
    int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= P) return;
    const double halfw = 0.5 * (double)w;
    int ix, iy;
    float fx, fy;
    cell_t12(x.p[0][j], h0, halfw, prec64, ix, fx);
    cell_t12(x.p[1][j], h1, halfw, prec64, iy, fy);
    word[j] = ym_word(pmod(ix, n0), pmod(iy, n1), n1 / kYmChunk, w);
    fro.p[0][j] = fx;
    fro.p[1][j] = fy;
}

struct T3Src {
    double C[3], gam[3], hd[3], D[3], nf2[3];
};

// Type-3 sources: xi = ((x - C)/gam)/hd + nf/2 (ref: gpu_t3.py:480-485),
// prephase angle sum_d D_d x_d summed left to right (ref: gpu_t3.py:486-488).
__global__ void k_t3_src(int64_t P, D3 x, Geom g, T3Src c, int isign, int prec_flags,
                         I3 i1o, F3 fro, uint32_t *__restrict__ key,
                         float2 *__restrict__ pre) {
    int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= P) return;
    const bool coords64 = prec_flags & 1, phases64 = prec_flags & 2;
    const double halfw = 0.5 * (double)g.w;
    uint32_t k = 0;
    double ang64 = 0.0;
    float ang32 = 0.0f;
#pragma unroll
    for (int d = 0; d < 3; ++d) {
        double xv = x.p[d][j];
        int ii;
        float f;
        if (coords64) {
            double xi = ((xv - c.C[d]) / c.gam[d]) / c.hd[d] + c.nf2[d];
            ii = (int)ceil(xi - halfw);
            f = (float)(xi - (double)ii);
        } else {
            float xi = (((float)xv - (float)c.C[d]) / (float)c.gam[d]) / (float)c.hd[d] +
                       (float)c.nf2[d];
            ii = (int)ceilf(xi - (float)halfw);
            f = xi - (float)ii;
        }
        i1o.p[d][j] = ii;
        fro.p[d][j] = f;
        k = k * (uint32_t)g.nb[d] + (uint32_t)bin_of(ii, g.w / 2, g.n[d], g.m[d]);
        if (phases64)
            ang64 = ang64 + c.D[d] * xv;
        else
            ang32 = ang32 + (float)c.D[d] * (float)xv;
    }
    key[j] = k;
    double th = (double)isign * (phases64 ? ang64 : (double)ang32);
    double sn, cs;
    sincos(th, &sn, &cs);
    pre[j] = make_float2((float)cs, (float)sn);
}

struct T3Trg {
    double D[3], hg[3], h2[3], C[3], nu2[3];
};

// Type-3 targets (ref: gpu_t3.py:357-377): theta = (s - D)*hg,
// lam = theta/h2 + n_up/2, i1/fr; post = exp(i isign sum_d C_d (s_d - D_d))
// / prod_d phihat(theta_d) with phihat by the 128-node quadrature
// (ref: sizing.py:74-85).
__global__ void k_t3_trg(int64_t M, D3 s, Geom g, T3Trg c, int isign, int prec_flags,
                         const double *__restrict__ quad, int nquad, I3 i1o, F3 fro,
                         uint32_t *__restrict__ key, float2 *__restrict__ post) {
    int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= M) return;
    const bool coords64 = prec_flags & 1, phases64 = prec_flags & 2;
    const double halfw = 0.5 * (double)g.w;
    const double *dq = quad, *fq = quad + nquad;
    uint32_t k = 0;
    double tdec = 1.0;
    double ang64 = 0.0;
    float ang32 = 0.0f;
#pragma unroll
    for (int d = 0; d < 3; ++d) {
        double sv = s.p[d][j];
        double th64;
        int ii;
        float f;
        if (coords64) {
            double th = (sv - c.D[d]) * c.hg[d];
            double lam = th / c.h2[d] + c.nu2[d];
            ii = (int)ceil(lam - halfw);
            f = (float)(lam - (double)ii);
            th64 = th;
        } else {
            float th = ((float)sv - (float)c.D[d]) * (float)c.hg[d];
            float lam = th / (float)c.h2[d] + (float)c.nu2[d];
            ii = (int)ceilf(lam - (float)halfw);
            f = lam - (float)ii;
            th64 = (double)th;
        }
        i1o.p[d][j] = ii;
        fro.p[d][j] = f;
        k = k * (uint32_t)g.nb[d] + (uint32_t)bin_of(ii, g.w / 2, g.n[d], g.m[d]);
        double acc = 0.0;
        for (int q = 0; q < nquad; ++q) acc += fq[q] * cos(th64 * dq[q]);
        tdec = tdec * (2.0 * acc);
        if (phases64)
            ang64 = ang64 + c.C[d] * (sv - c.D[d]);
        else
            ang32 = ang32 + (float)c.C[d] * ((float)sv - (float)c.D[d]);
    }
    key[j] = k;
    double th = (double)isign * (phases64 ? ang64 : (double)ang32);
    double sn, cs;
    sincos(th, &sn, &cs);
    post[j] = make_float2((float)(cs / tdec), (float)(sn / tdec));
}

template <int DIM>
__global__ void k_gather_points(int64_t P, const uint32_t *__restrict__ perm, CI3 i1i, CF3 fri,
                                I3 i1o, F3 fro, const float2 *__restrict__ xin,
                                float2 *__restrict__ xout) {
    int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= P) return;
    uint32_t src = perm[j];
#pragma unroll
    for (int d = 0; d < DIM; ++d) {
        i1o.p[d][j] = i1i.p[d][src];
        fro.p[d][j] = fri.p[d][src];
    }
    if (xin) xout[j] = xin[src];
}

__global__ void k_permute_c64(int64_t P, const uint32_t *__restrict__ perm,
                              const float2 *__restrict__ in, float2 *__restrict__ out) {
    int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j < P) out[j] = in[perm[j]];
}

inline unsigned blocks_for(int64_t n, int t) { return (unsigned)((n + t - 1) / t); }

}  // namespace
}  // namespace mn

using namespace mn;

extern "C" {

int mn_setpts_t12(const mn_bins *g, int64_t P, const double *const x[3], int prec64,
                  int32_t *const i1[3], float *const fr[3], uint32_t *key,
                  mn_stream_t stream) {
    clear_error();
    int rc = check_bins(g);
    if (rc) return rc;
    MN_REQUIRE(P >= 1 && P < (int64_t(1) << 32), "setpts: P must be in [1, 2^32)");
    MN_REQUIRE(key != nullptr, "setpts: key is NULL");
    D3 xs{};
    I3 io{};
    F3 fo{};
    double h[3] = {1.0, 1.0, 1.0};
    for (int d = 0; d < g->dim; ++d) {
        MN_REQUIRE(x[d] && i1[d] && fr[d], "setpts: NULL coordinate/output pointer");
        xs.p[d] = x[d];
        io.p[d] = i1[d];
        fo.p[d] = fr[d];
        h[d] = kTwoPi / (double)g->n[d];  // same fp64 value as 2*pi/n_up on the host
    }
    Geom k = make_geom(g);
    hipStream_t s = as_stream(stream);
    unsigned nb = blocks_for(P, 256);
    switch (g->dim) {
        case 1: k_setpts_t12<1><<<nb, 256, 0, s>>>(P, xs, k, h[0], h[1], h[2], prec64, io, fo, key); break;
        case 2: k_setpts_t12<2><<<nb, 256, 0, s>>>(P, xs, k, h[0], h[1], h[2], prec64, io, fo, key); break;
        default: k_setpts_t12<3><<<nb, 256, 0, s>>>(P, xs, k, h[0], h[1], h[2], prec64, io, fo, key); break;
    }
    MN_LAUNCH_CHECK("setpts_t12");
    return MN_OK;
}

static int zs_setpts(bool gather, const mn_bins *g, int64_t P, const double *const x[3],
                     int prec64, uint32_t *word, float *const fr[3], mn_stream_t stream) {
    clear_error();
    int rc = zsweep_check(g);
    if (rc) return rc;
    MN_REQUIRE(P >= 1 && P < (int64_t(1) << 31), "zsweep setpts: P must be in [1, 2^31)");
    MN_REQUIRE(x && fr && word, "zsweep setpts: NULL pointer");
    D3 xs{};
    F3 fo{};
    double h[3];
    for (int d = 0; d < 3; ++d) {
        MN_REQUIRE(x[d] && fr[d], "zsweep setpts: NULL coordinate/output pointer");
        xs.p[d] = x[d];
        fo.p[d] = fr[d];
        h[d] = kTwoPi / (double)g->n[d];
    }
    auto kern = gather ? k_zs_setpts<true> : k_zs_setpts<false>;
    kern<<<blocks_for(P, ZP_THREADS * ZP_ITEMS), ZP_THREADS, 0, as_stream(stream)>>>(
        P, xs, (int)g->n[0], (int)g->n[1], (int)g->n[2], g->w, h[0], h[1], h[2], prec64, word, fo);
    MN_LAUNCH_CHECK("zsweep_setpts");
    return MN_OK;
}

int mn_zsweep_setpts(const mn_bins *g, int64_t P, const double *const x[3], int prec64,
                     uint32_t *word, float *const fr[3], mn_stream_t stream) {
    return zs_setpts(false, g, P, x, prec64, word, fr, stream);
}

int mn_zgather_setpts(const mn_bins *g, int64_t P, const double *const x[3], int prec64,
                      uint32_t *word, float *const fr[3], mn_stream_t stream) {
    return zs_setpts(true, g, P, x, prec64, word, fr, stream);
}

int mn_ysweep_setpts(const mn_bins *g, int64_t P, const double *const x[2], int prec64,
                     uint32_t *word, float *const fr[2], mn_stream_t stream) {
    clear_error();
    int rc = ysweep_check(g);
    if (rc) return rc;
    MN_REQUIRE(P >= 1 && P < (int64_t(1) << 31), "ysweep setpts: P must be in [1, 2^31)");
    MN_REQUIRE(x && fr && word, "ysweep setpts: NULL pointer");
    D3 xs{};
    F3 fo{};
    for (int d = 0; d < 2; ++d) {
        MN_REQUIRE(x[d] && fr[d], "ysweep setpts: NULL coordinate/output pointer");
        xs.p[d] = x[d];
        fo.p[d] = fr[d];
    }
    k_ys_setpts<<<blocks_for(P, 256), 256, 0, as_stream(stream)>>>(
        P, xs, (int)g->n[0], (int)g->n[1], g->w, kTwoPi / (double)g->n[0],
        kTwoPi / (double)g->n[1], prec64, word, fo);
    MN_LAUNCH_CHECK("ysweep_setpts");
    return MN_OK;
}

int mn_ymfma_setpts(const mn_bins *g, int64_t P, const double *const x[2], int prec64,
                    uint32_t *word, float *const fr[2], mn_stream_t stream) {
    clear_error();
    int rc = ymfma_check(g);
    if (rc) return rc;
    MN_REQUIRE(P >= 1 && P < (int64_t(1) << 31), "ymfma setpts: P must be in [1, 2^31)");
    MN_REQUIRE(x && fr && word, "ymfma setpts: NULL pointer");
    D3 xs{};
    F3 fo{};
    for (int d = 0; d < 2; ++d) {
        MN_REQUIRE(x[d] && fr[d], "ymfma setpts: NULL coordinate/output pointer");
        xs.p[d] = x[d];
        fo.p[d] = fr[d];
    }
    k_ym_setpts<<<blocks_for(P, 256), 256, 0, as_stream(stream)>>>(
        P, xs, (int)g->n[0], (int)g->n[1], g->w, kTwoPi / (double)g->n[0],
        kTwoPi / (double)g->n[1], prec64, word, fo);
    MN_LAUNCH_CHECK("ymfma_setpts");
    return MN_OK;
}

int mn_permute_c64(int64_t P, const uint32_t *perm, const void *in, void *out,
                   mn_stream_t stream) {
    clear_error();
    MN_REQUIRE(P >= 1 && P < (int64_t(1) << 32), "permute: P must be in [1, 2^32)");
    MN_REQUIRE(perm && in && out && in != out, "permute: NULL or aliased pointer");
    k_permute_c64<<<blocks_for(P, 256), 256, 0, as_stream(stream)>>>(
        P, perm, static_cast<const float2 *>(in), static_cast<float2 *>(out));
    MN_LAUNCH_CHECK("permute_c64");
    return MN_OK;
}

int mn_t3_setpts_src(const mn_bins *g, int64_t P, const double *const x[3], const double C[3],
                     const double gam[3], const double hd[3], const double D[3], int isign,
                     int prec_flags, int32_t *const i1[3], float *const fr[3], uint32_t *key,
                     void *pre, mn_stream_t stream) {
    clear_error();
    int rc = check_bins(g);
    if (rc) return rc;
    MN_REQUIRE(g->dim == 3, "t3 setpts: geometry must be 3D");
    MN_REQUIRE(P >= 1 && P < (int64_t(1) << 32), "t3 setpts: P must be in [1, 2^32)");
    MN_REQUIRE(key && pre, "t3 setpts: NULL output");
    D3 xs{};
    I3 io{};
    F3 fo{};
    T3Src c{};
    for (int d = 0; d < 3; ++d) {
        MN_REQUIRE(x[d] && i1[d] && fr[d], "t3 setpts: NULL coordinate/output pointer");
        xs.p[d] = x[d];
        io.p[d] = i1[d];
        fo.p[d] = fr[d];
        c.C[d] = C[d];
        c.gam[d] = gam[d];
        c.hd[d] = hd[d];
        c.D[d] = D[d];
        c.nf2[d] = (double)g->n[d] / 2.0;
    }
    Geom k = make_geom(g);
    hipStream_t s = as_stream(stream);
    k_t3_src<<<blocks_for(P, 256), 256, 0, s>>>(P, xs, k, c, isign >= 0 ? 1 : -1, prec_flags,
                                                io, fo, key, static_cast<float2 *>(pre));
    MN_LAUNCH_CHECK("t3_setpts_src");
    return MN_OK;
}

int mn_t3_setpts_trg(const mn_bins *g, int64_t M, const double *const s[3], const double D[3],
                     const double hg[3], const double h2[3], const double C[3], int isign,
                     int prec_flags, const double *quad, int nquad, int32_t *const i1[3],
                     float *const fr[3], uint32_t *key, void *post, mn_stream_t stream) {
    clear_error();
    int rc = check_bins(g);
    if (rc) return rc;
    MN_REQUIRE(g->dim == 3, "t3 targets: geometry must be 3D");
    MN_REQUIRE(M >= 1 && M < (int64_t(1) << 32), "t3 targets: M must be in [1, 2^32)");
    MN_REQUIRE(key && post && quad && nquad >= 1, "t3 targets: NULL output or quadrature");
    D3 ss{};
    I3 io{};
    F3 fo{};
    T3Trg c{};
    for (int d = 0; d < 3; ++d) {
        MN_REQUIRE(s[d] && i1[d] && fr[d], "t3 targets: NULL coordinate/output pointer");
        ss.p[d] = s[d];
        io.p[d] = i1[d];
        fo.p[d] = fr[d];
        c.D[d] = D[d];
        c.hg[d] = hg[d];
        c.h2[d] = h2[d];
        c.C[d] = C[d];
        c.nu2[d] = (double)g->n[d] / 2.0;
    }
    Geom k = make_geom(g);
    hipStream_t st = as_stream(stream);
    k_t3_trg<<<blocks_for(M, 256), 256, 0, st>>>(M, ss, k, c, isign >= 0 ? 1 : -1, prec_flags,
                                                 quad, nquad, io, fo, key,
                                                 static_cast<float2 *>(post));
    MN_LAUNCH_CHECK("t3_setpts_trg");
    return MN_OK;
}

int mn_gather_points(int dim, int64_t P, const uint32_t *perm, const int32_t *const i1_in[3],
                     const float *const fr_in[3], int32_t *const i1_out[3],
                     float *const fr_out[3], const void *extra_in, void *extra_out,
                     mn_stream_t stream) {
    clear_error();
    MN_REQUIRE(dim >= 1 && dim <= 3, "gather_points: dim must be 1, 2 or 3");
    MN_REQUIRE(P >= 1 && perm, "gather_points: bad P or NULL perm");
    MN_REQUIRE((extra_in == nullptr) == (extra_out == nullptr),
               "gather_points: extra_in/extra_out must both be set or both NULL");
    CI3 ii{};
    CF3 fi{};
    I3 io{};
    F3 fo{};
    for (int d = 0; d < dim; ++d) {
        MN_REQUIRE(i1_in[d] && fr_in[d] && i1_out[d] && fr_out[d], "gather_points: NULL pointer");
        ii.p[d] = i1_in[d];
        fi.p[d] = fr_in[d];
        io.p[d] = i1_out[d];
        fo.p[d] = fr_out[d];
    }
    hipStream_t s = as_stream(stream);
    unsigned nb = blocks_for(P, 256);
    const float2 *xi = static_cast<const float2 *>(extra_in);
    float2 *xo = static_cast<float2 *>(extra_out);
    switch (dim) {
        case 1: k_gather_points<1><<<nb, 256, 0, s>>>(P, perm, ii, fi, io, fo, xi, xo); break;
        case 2: k_gather_points<2><<<nb, 256, 0, s>>>(P, perm, ii, fi, io, fo, xi, xo); break;
        default: k_gather_points<3><<<nb, 256, 0, s>>>(P, perm, ii, fi, io, fo, xi, xo); break;
    }
    MN_LAUNCH_CHECK("gather_points");
    return MN_OK;
}

}  // extern "C"
