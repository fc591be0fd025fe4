/*
 * CPU oracle for the MI355X NUFFT engine -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker / the reported CPU baseline.
 * The product (mlx_nufft_amd) never calls it.
 *
 * Plain-C restatement of the reference algorithm (mlx-nufft) for the hot
 * path, written from the reference's Python/numpy source and the
 * mathematics of the transforms:
 *   or_setpts_t12    crit64 fold + rescale        (ref: nd.py:152-165)
 *   or_bin_keys      bin key of the engine's bins  (ref: nd.py:308-313)
 *   or_stable_sort   stable counting sort          (ref: nd.py:314)
 *   or_spread        fp64 ES spread, periodic      (ref: nd.py:437-579)
 *   or_interp        fp64 ES interpolation         (ref: nd.py:908-1073)
 *   or_spread_f32    OpenMP fp32 spread (the CPU-baseline port)
 *   or_dft_t1        exact fp64 type-1 sums on a tensor grid of modes
 *   or_dft_t2        exact fp64 type-2 sums at selected points
 *   or_dft_t3        exact fp64 type-3 sums at selected targets
 *                    (ref: harness/gen.py:93-114, direct_sum)
 * Build: gcc -O2 -fopenmp -ffp-contract=off -shared -fPIC (oracle/Makefile).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define TWO_PI 6.283185307179586 /* fl64(2*pi) == 2.0*np.pi */

/* np.mod(x, 2pi) for float64: fmod, then a negative remainder moves up by
 * 2pi; a zero remainder becomes +0. */
static double np_mod_2pi(double x) {
    double r = fmod(x, TWO_PI);
    if (r != 0.0) {
        if (r < 0.0) r += TWO_PI;
    } else {
        r = 0.0;
    }
    return r;
}

static int64_t pmod64(int64_t v, int64_t n) {
    int64_t r = v % n;
    return r < 0 ? r + n : r;
}

/* ES kernel psi(d) = exp(beta*(sqrt(1-(2d/w)^2)-1)), 0 outside |d| <= w/2
 * (ref: sizing.py:53-62). */
static double es(double d, double beta, int w) {
    double z = 2.0 * d / (double)w;
    double z2 = z * z;
    if (z2 > 1.0) return 0.0;
    return exp(beta * (sqrt(1.0 - z2) - 1.0));
}

void or_setpts_t12(int dim, int64_t P, const double *const *x, const int64_t *n, int w,
                   int prec64, int32_t *const *i1, float *const *fr) {
    for (int d = 0; d < dim; ++d) {
        const double h = TWO_PI / (double)n[d];
        const double halfw = (double)w / 2.0;
#pragma omp parallel for schedule(static)
        for (int64_t j = 0; j < P; ++j) {
            double r = np_mod_2pi(x[d][j]);
            if (prec64) {
                double xi = r / h;
                int32_t ii = (int32_t)ceil(xi - halfw);
                i1[d][j] = ii;
                fr[d][j] = (float)(xi - (double)ii);
            } else {
                float xi = (float)r / (float)h;
                int32_t ii = (int32_t)ceilf(xi - (float)halfw);
                i1[d][j] = ii;
                fr[d][j] = xi - (float)ii;
            }
        }
    }
}

/* Bin of a point: b_d = ((i1_d + w/2) mod n_d) / m_d, key row-major over nb. */
void or_bin_keys(int dim, int64_t P, const int32_t *const *i1, const int64_t *n,
                 const int32_t *m, const int32_t *nb, int w, uint32_t *key) {
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < P; ++j) {
        uint64_t k = 0;
        for (int d = 0; d < dim; ++d) {
            int64_t v = pmod64((int64_t)i1[d][j] + w / 2, n[d]);
            k = k * (uint64_t)nb[d] + (uint64_t)(v / m[d]);
        }
        key[j] = (uint32_t)k;
    }
}

/* Stable counting sort: perm[r] = index of the r-th smallest key, ties in
 * index order (== numpy argsort(kind="stable")). Returns 0, or -1 if a key
 * is >= nkeys or memory runs out. */
int or_stable_sort(int64_t P, const uint32_t *key, int64_t nkeys, uint32_t *perm) {
    int64_t *cnt = (int64_t *)calloc((size_t)nkeys + 1, sizeof(int64_t));
    if (!cnt) return -1;
    for (int64_t j = 0; j < P; ++j) {
        if ((int64_t)key[j] >= nkeys) {
            free(cnt);
            return -1;
        }
        cnt[key[j] + 1]++;
    }
    for (int64_t k = 0; k < nkeys; ++k) cnt[k + 1] += cnt[k];
    for (int64_t j = 0; j < P; ++j) perm[cnt[key[j]]++] = (uint32_t)j;
    free(cnt);
    return 0;
}

/* Weight precision of taps(): 0 = fp64 ES kernel; 1 = the fp32 evaluation
 * exp2(beta log2(e) (sqrt(max(1 - z^2, 0)) - 1)) with z = (a - fr) (2/w),
 * every step rounded to fp32 (a CPU emulation: the GPU's hardware exp2/sqrt
 * carry about 1 ulp of their own); 2 = the same in fp32 with the exponent
 * written -beta log2(e) z^2 / (1 + sqrt(1 - z^2)). Products and sums stay
 * fp64 either way. Test infrastructure, set per process. */
static int g_weights_f32 = 0;

void or_set_weights_f32(int mode) { g_weights_f32 = mode; }

static double es_f32(float d, double beta, int w) {
    const float z = d * (2.0f / (float)w);
    const float t = fmaxf(1.0f - z * z, 0.0f);
    const float bl2e = (float)(beta * 1.4426950408889634);
    if (g_weights_f32 == 2)  /* sqrt(t) - 1 = -z^2 / (1 + sqrt(t)): no cancellation */
        return (double)exp2f(-bl2e * (z * z) / (1.0f + sqrtf(t)));
    return (double)exp2f(bl2e * (sqrtf(t) - 1.0f));
}

/* Taps of one point along one dim: wrapped cell indices and ES weights. */
static void taps(int32_t i1, float fr, int64_t n, int w, double beta, int64_t *cell,
                 double *wt) {
    for (int a = 0; a < w; ++a) {
        cell[a] = pmod64((int64_t)i1 + a, n);
        wt[a] = g_weights_f32 ? es_f32((float)a - fr, beta, w)
                              : es((double)a - (double)fr, beta, w);
    }
}

/* grid[cell] += c_j * prod_d psi(a_d - fr_d) over the w^dim taps of every
 * point (grid: prod n complex128, interleaved, accumulated into). */
void or_spread(int dim, int64_t P, const int32_t *const *i1, const float *const *fr,
               const double *c, const int64_t *n, int w, double beta, double *grid) {
    int64_t n1 = dim >= 2 ? n[1] : 1, n2 = dim >= 3 ? n[2] : 1;
    int64_t cx[16], cy[16], cz[16];
    double wx[16], wy[16], wz[16];
    for (int a = 0; a < 16; ++a) {
        cy[a] = cz[a] = 0;
        wy[a] = wz[a] = 1.0;
    }
    int wy_n = dim >= 2 ? w : 1, wz_n = dim >= 3 ? w : 1;
    for (int64_t j = 0; j < P; ++j) {
        taps(i1[0][j], fr[0][j], n[0], w, beta, cx, wx);
        if (dim >= 2) taps(i1[1][j], fr[1][j], n[1], w, beta, cy, wy);
        if (dim >= 3) taps(i1[2][j], fr[2][j], n[2], w, beta, cz, wz);
        const double cr = c[2 * j], ci = c[2 * j + 1];
        for (int a = 0; a < w; ++a)
            for (int b = 0; b < wy_n; ++b)
                for (int e = 0; e < wz_n; ++e) {
                    double v = wx[a] * wy[b] * wz[e];
                    int64_t cell = (cx[a] * n1 + cy[b]) * n2 + cz[e];
                    grid[2 * cell] += cr * v;
                    grid[2 * cell + 1] += ci * v;
                }
    }
}

/* out_j = sum over taps of grid[cell] * prod_d psi(a_d - fr_d) (complex128). */
void or_interp(int dim, int64_t P, const int32_t *const *i1, const float *const *fr,
               const double *grid, const int64_t *n, int w, double beta, double *out) {
    int64_t n1 = dim >= 2 ? n[1] : 1, n2 = dim >= 3 ? n[2] : 1;
    int wy_n = dim >= 2 ? w : 1, wz_n = dim >= 3 ? w : 1;
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < P; ++j) {
        int64_t cx[16], cy[16], cz[16];
        double wx[16], wy[16], wz[16];
        for (int a = 0; a < 16; ++a) {
            cy[a] = cz[a] = 0;
            wy[a] = wz[a] = 1.0;
        }
        taps(i1[0][j], fr[0][j], n[0], w, beta, cx, wx);
        if (dim >= 2) taps(i1[1][j], fr[1][j], n[1], w, beta, cy, wy);
        if (dim >= 3) taps(i1[2][j], fr[2][j], n[2], w, beta, cz, wz);
        double sr = 0.0, si = 0.0;
        for (int a = 0; a < w; ++a)
            for (int b = 0; b < wy_n; ++b)
                for (int e = 0; e < wz_n; ++e) {
                    double v = wx[a] * wy[b] * wz[e];
                    int64_t cell = (cx[a] * n1 + cy[b]) * n2 + cz[e];
                    sr += grid[2 * cell] * v;
                    si += grid[2 * cell + 1] * v;
                }
        out[2 * j] = sr;
        out[2 * j + 1] = si;
    }
}

/* CPU-baseline spread in fp32 with OpenMP: points are bucketed into slabs
 * of `slab` rows of dim 0 (slab >= w); slabs of one colour never share grid
 * rows, so each colour runs in parallel without atomics (two colours, plus a
 * third for the last slab when the slab count is odd). c: complex64
 * interleaved, caller order; grid: complex64, overwritten. */
int or_spread_f32(int dim, int64_t P, const int32_t *const *i1, const float *const *fr,
                  const float *c, const int64_t *n, int w, double beta, int64_t slab,
                  float *grid) {
    int64_t n0 = n[0], n1 = dim >= 2 ? n[1] : 1, n2 = dim >= 3 ? n[2] : 1;
    memset(grid, 0, sizeof(float) * 2 * (size_t)(n0 * n1 * n2));
    if (slab < w) slab = w;
    /* floor: the last slab absorbs the remainder, so every slab is >= w rows */
    int64_t ns = n0 / slab;
    if (ns < 3) ns = 1, slab = n0;
    int64_t *cnt = (int64_t *)calloc((size_t)ns + 1, sizeof(int64_t));
    int64_t *idx = (int64_t *)malloc(sizeof(int64_t) * (size_t)P);
    if (!cnt || !idx) {
        free(cnt);
        free(idx);
        return -1;
    }
#define SLAB_OF(j) ((pmod64((int64_t)i1[0][j] + w / 2, n0) / slab) < ns - 1 \
                        ? (pmod64((int64_t)i1[0][j] + w / 2, n0) / slab) : ns - 1)
    for (int64_t j = 0; j < P; ++j) cnt[SLAB_OF(j) + 1]++;
    for (int64_t s = 0; s < ns; ++s) cnt[s + 1] += cnt[s];
    {
        int64_t *pos = (int64_t *)malloc(sizeof(int64_t) * (size_t)ns);
        memcpy(pos, cnt, sizeof(int64_t) * (size_t)ns);
        for (int64_t j = 0; j < P; ++j) idx[pos[SLAB_OF(j)]++] = j;
        free(pos);
    }
    const float bl = (float)beta, inv = 2.0f / (float)w;
    int wy_n = dim >= 2 ? w : 1, wz_n = dim >= 3 ? w : 1;
    int ncol = (ns == 1) ? 1 : ((ns % 2) ? 3 : 2);
    for (int col = 0; col < ncol; ++col) {
#pragma omp parallel for schedule(dynamic, 1)
        for (int64_t s = 0; s < ns; ++s) {
            int scol = (ncol == 3 && s == ns - 1) ? 2 : (int)(s % 2);
            if (ncol == 1) scol = 0;
            if (scol != col) continue;
            for (int64_t q = cnt[s]; q < cnt[s + 1]; ++q) {
                int64_t j = idx[q];
                float wx[16], wy[16], wz[16];
                int64_t cx[16], cy[16], cz[16];
                for (int a = 0; a < 16; ++a) {
                    cy[a] = cz[a] = 0;
                    wy[a] = wz[a] = 1.0f;
                }
                for (int d = 0; d < dim; ++d) {
                    float *wd = d == 0 ? wx : (d == 1 ? wy : wz);
                    int64_t *cd = d == 0 ? cx : (d == 1 ? cy : cz);
                    for (int a = 0; a < w; ++a) {
                        float z = ((float)a - fr[d][j]) * inv;
                        float t = 1.0f - z * z;
                        wd[a] = t > 0.0f ? expf(bl * (sqrtf(t) - 1.0f)) : 0.0f;
                        cd[a] = pmod64((int64_t)i1[d][j] + a, n[d]);
                    }
                }
                const float cr = c[2 * j], ci = c[2 * j + 1];
                for (int a = 0; a < w; ++a)
                    for (int b = 0; b < wy_n; ++b) {
                        const float wab = wx[a] * wy[b];
                        const float vr = cr * wab, vi = ci * wab;
                        float *row = grid + 2 * ((cx[a] * n1 + cy[b]) * n2);
                        for (int e = 0; e < wz_n; ++e) {
                            row[2 * cz[e]] += vr * wz[e];
                            row[2 * cz[e] + 1] += vi * wz[e];
                        }
                    }
            }
        }
    }
    free(cnt);
    free(idx);
    return 0;
}

/* f[a,b,e] = sum_j c_j exp(i*isign*(k0[a] x0_j + k1[b] x1_j + k2[e] x2_j))
 * for the tensor grid of integer modes k0 x k1 x k2 (dims beyond `dim` use
 * nk = 1, k = 0). out: complex128 nk0*nk1*nk2, C order. */
void or_dft_t1(int dim, int64_t P, const double *const *x, const double *c, const int64_t *nk,
               const int64_t *const *k, int isign, double *out) {
    const int64_t K0 = nk[0], K1 = dim >= 2 ? nk[1] : 1, K2 = dim >= 3 ? nk[2] : 1;
    const int64_t NK = K0 * K1 * K2;
    memset(out, 0, sizeof(double) * 2 * (size_t)NK);
#pragma omp parallel
    {
        double *acc = (double *)calloc(2 * (size_t)NK, sizeof(double));
        double *e0 = (double *)malloc(sizeof(double) * 2 * (size_t)K0);
        double *e1 = (double *)malloc(sizeof(double) * 2 * (size_t)K1);
        double *e2 = (double *)malloc(sizeof(double) * 2 * (size_t)K2);
#pragma omp for schedule(static)
        for (int64_t j = 0; j < P; ++j) {
            for (int64_t a = 0; a < K0; ++a) {
                double ph = (double)isign * (double)k[0][a] * x[0][j];
                e0[2 * a] = cos(ph);
                e0[2 * a + 1] = sin(ph);
            }
            for (int64_t b = 0; b < K1; ++b) {
                double ph = dim >= 2 ? (double)isign * (double)k[1][b] * x[1][j] : 0.0;
                e1[2 * b] = cos(ph);
                e1[2 * b + 1] = sin(ph);
            }
            for (int64_t e = 0; e < K2; ++e) {
                double ph = dim >= 3 ? (double)isign * (double)k[2][e] * x[2][j] : 0.0;
                e2[2 * e] = cos(ph);
                e2[2 * e + 1] = sin(ph);
            }
            const double cr = c[2 * j], ci = c[2 * j + 1];
            for (int64_t a = 0; a < K0; ++a) {
                double ar = cr * e0[2 * a] - ci * e0[2 * a + 1];
                double ai = cr * e0[2 * a + 1] + ci * e0[2 * a];
                for (int64_t b = 0; b < K1; ++b) {
                    double br = ar * e1[2 * b] - ai * e1[2 * b + 1];
                    double bi = ar * e1[2 * b + 1] + ai * e1[2 * b];
                    double *o = acc + 2 * ((a * K1 + b) * K2);
                    for (int64_t e = 0; e < K2; ++e) {
                        o[2 * e] += br * e2[2 * e] - bi * e2[2 * e + 1];
                        o[2 * e + 1] += br * e2[2 * e + 1] + bi * e2[2 * e];
                    }
                }
            }
        }
#pragma omp critical
        for (int64_t q = 0; q < 2 * NK; ++q) out[q] += acc[q];
        free(acc);
        free(e0);
        free(e1);
        free(e2);
    }
}

/* c_j = sum_k f[k] exp(i*isign*k.x_j) over the full modeord=0 box N (f:
 * complex128 C order) at the points listed in jidx (nj of them). */
void or_dft_t2(int dim, const double *const *x, const double *f, const int64_t *N, int isign,
               int64_t nj, const int64_t *jidx, double *out) {
    const int64_t N0 = N[0], N1 = dim >= 2 ? N[1] : 1, N2 = dim >= 3 ? N[2] : 1;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t q = 0; q < nj; ++q) {
        const int64_t j = jidx[q];
        double *e0 = (double *)malloc(sizeof(double) * 2 * (size_t)N0);
        double *e1 = (double *)malloc(sizeof(double) * 2 * (size_t)N1);
        double *e2 = (double *)malloc(sizeof(double) * 2 * (size_t)N2);
        for (int64_t a = 0; a < N0; ++a) {
            double ph = (double)isign * (double)(a - N0 / 2) * x[0][j];
            e0[2 * a] = cos(ph);
            e0[2 * a + 1] = sin(ph);
        }
        for (int64_t b = 0; b < N1; ++b) {
            double ph = dim >= 2 ? (double)isign * (double)(b - N1 / 2) * x[1][j] : 0.0;
            e1[2 * b] = cos(ph);
            e1[2 * b + 1] = sin(ph);
        }
        for (int64_t e = 0; e < N2; ++e) {
            double ph = dim >= 3 ? (double)isign * (double)(e - N2 / 2) * x[2][j] : 0.0;
            e2[2 * e] = cos(ph);
            e2[2 * e + 1] = sin(ph);
        }
        double sr = 0.0, si = 0.0;
        for (int64_t a = 0; a < N0; ++a) {
            double tr = 0.0, ti = 0.0;
            for (int64_t b = 0; b < N1; ++b) {
                double ur = 0.0, ui = 0.0;
                const double *fr = f + 2 * ((a * N1 + b) * N2);
                for (int64_t e = 0; e < N2; ++e) {
                    ur += fr[2 * e] * e2[2 * e] - fr[2 * e + 1] * e2[2 * e + 1];
                    ui += fr[2 * e] * e2[2 * e + 1] + fr[2 * e + 1] * e2[2 * e];
                }
                tr += ur * e1[2 * b] - ui * e1[2 * b + 1];
                ti += ur * e1[2 * b + 1] + ui * e1[2 * b];
            }
            sr += tr * e0[2 * a] - ti * e0[2 * a + 1];
            si += tr * e0[2 * a + 1] + ti * e0[2 * a];
        }
        out[2 * q] = sr;
        out[2 * q + 1] = si;
        free(e0);
        free(e1);
        free(e2);
    }
}

/* f_k = sum_j c_j exp(i*isign*s_k.x_j) (3D) at the targets listed in kidx. */
void or_dft_t3(int64_t P, const double *const *x, const double *c, const double *const *s,
               int isign, int64_t nk, const int64_t *kidx, double *out) {
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t q = 0; q < nk; ++q) {
        const int64_t k = kidx[q];
        double sr = 0.0, si = 0.0;
        for (int64_t j = 0; j < P; ++j) {
            double ph = (double)isign * (s[0][k] * x[0][j] + s[1][k] * x[1][j] + s[2][k] * x[2][j]);
            double cs = cos(ph), sn = sin(ph);
            sr += c[2 * j] * cs - c[2 * j + 1] * sn;
            si += c[2 * j] * sn + c[2 * j + 1] * cs;
        }
        out[2 * q] = sr;
        out[2 * q + 1] = si;
    }
}
