// Pruned, deconvolving multi-dimensional FFT for power-of-two fine grids.
//
// Type 1 needs only the N_d lowest modes of each axis of the n_d-point
// transform of the spread grid, each multiplied by its deconvolution factor;
// type 2 needs the transform of a grid that is zero outside those modes.
// Instead of a full 3D FFT (four rocFFT passes over the whole grid) plus a
// crop kernel, one pass per axis transforms the lines of that axis and
// keeps (type 1) or fills (type 2) only the N_d modes, fusing dec_d:
//
//   type 1:  grid (n0 n1 n2) -z-> (n0 n1 N2) -y-> (n0 N1 N2) -x-> fk (N0 N1 N2)
//   type 2:  fk -x-> (n0 N1 N2) -y-> (n0 n1 N2) -z-> grid (n0 n1 n2)
//
// which at n = 2N moves 2.6x fewer bytes than FFT + crop.
//
// One workgroup transforms TI lines of length n = 2^LOGN in LDS with
// Stockham radix-8 stages (one radix-2 or radix-4 stage when LOGN is not a
// multiple of 3); the output is in natural order. Lines are indexed
// (outer, inner) with element l of a line at (outer*L + l)*inner + inner_idx,
// so a tile of TI consecutive lines reads TI contiguous values per l when
// the axis is strided (inner >= TI) and TI contiguous lines when it is the
// last axis (inner == 1). Twiddles exp(+-2 pi i m/n) are rounded from fp64
// once per workgroup into LDS.
//
// ref: nd.py:374-383 (_fft_grid: per-axis MLX FFTs of the whole grid),
// nd.py:416-435 (crop + deconvolution kernel), nd.py:878-906 (type-2 pad +
// deconvolution), gpu_t3.py:94-148 (fft_axis).
#include "mn_common.h"

namespace mn {
namespace {

constexpr int FP_THREADS = 256;
constexpr int FP_ELEMS = 8192;  // complex values per workgroup tile (64 KB)

__device__ __forceinline__ float2 cadd(float2 a, float2 b) { return make_float2(a.x + b.x, a.y + b.y); }
__device__ __forceinline__ float2 csub(float2 a, float2 b) { return make_float2(a.x - b.x, a.y - b.y); }
__device__ __forceinline__ float2 cmul(float2 a, float2 b) {
    return make_float2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}
// a * (S i)
template <int S>
__device__ __forceinline__ float2 mul_si(float2 a) {
    return S > 0 ? make_float2(-a.y, a.x) : make_float2(a.y, -a.x);
}

// In-register DFTs X[k] = sum_m v[m] exp(S 2 pi i m k / R).
template <int S>
__device__ __forceinline__ void dft2(float2 *v) {
    const float2 a = v[0];
    v[0] = cadd(a, v[1]);
    v[1] = csub(a, v[1]);
}

template <int S>
__device__ __forceinline__ void dft4(float2 &v0, float2 &v1, float2 &v2, float2 &v3) {
    const float2 a0 = cadd(v0, v2), a1 = csub(v0, v2), a2 = cadd(v1, v3);
    const float2 a3 = mul_si<S>(csub(v1, v3));
    v0 = cadd(a0, a2);
    v2 = csub(a0, a2);
    v1 = cadd(a1, a3);
    v3 = csub(a1, a3);
}

template <int S>
__device__ __forceinline__ void dft4(float2 *v) { dft4<S>(v[0], v[1], v[2], v[3]); }

template <int S>
__device__ __forceinline__ void dft8(float2 *v) {
    constexpr float R2 = 0.70710678118654752f;
    float2 e0 = v[0], e1 = v[2], e2 = v[4], e3 = v[6];
    float2 o0 = v[1], o1 = v[3], o2 = v[5], o3 = v[7];
    dft4<S>(e0, e1, e2, e3);
    dft4<S>(o0, o1, o2, o3);
    // o_k *= exp(S i pi k / 4)
    o1 = make_float2((o1.x - S * o1.y) * R2, (o1.y + S * o1.x) * R2);
    o2 = mul_si<S>(o2);
    o3 = make_float2((-o3.x - S * o3.y) * R2, (-o3.y + S * o3.x) * R2);
    v[0] = cadd(e0, o0);
    v[4] = csub(e0, o0);
    v[1] = cadd(e1, o1);
    v[5] = csub(e1, o1);
    v[2] = cadd(e2, o2);
    v[6] = csub(e2, o2);
    v[3] = cadd(e3, o3);
    v[7] = csub(e3, o3);
}

template <int R, int S>
__device__ __forceinline__ void dft(float2 *v) {
    if constexpr (R == 8) dft8<S>(v);
    else if constexpr (R == 4) dft4<S>(v);
    else dft2<S>(v);
}

// One Stockham stage of radix R over TI lines of length N in buf
// (element l of line t at buf[l*TI + t]); Ns = product of the radices of
// the earlier stages. tw[m] = exp(S 2 pi i m / N).
template <int N, int TI, int R, int S>
__device__ __forceinline__ void stage(float2 *buf, const float2 *tw, int Ns) {
    constexpr int NB = (N / R) * TI;  // butterflies in the tile
    constexpr int MB = (NB + FP_THREADS - 1) / FP_THREADS;
    float2 v[MB][R];
#pragma unroll
    for (int m = 0; m < MB; ++m) {
        const int b = threadIdx.x + m * FP_THREADS;
        if (b < NB) {
            const int t = b % TI, j = b / TI, k = j & (Ns - 1);
            const int tstep = N / (Ns * R);
#pragma unroll
            for (int r = 0; r < R; ++r) v[m][r] = buf[(j + r * (N / R)) * TI + t];
            if (Ns > 1) {
#pragma unroll
                for (int r = 1; r < R; ++r) v[m][r] = cmul(v[m][r], tw[k * r * tstep]);
            }
            dft<R, S>(v[m]);
        }
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < MB; ++m) {
        const int b = threadIdx.x + m * FP_THREADS;
        if (b < NB) {
            const int t = b % TI, j = b / TI, k = j & (Ns - 1);
            const int base = (j - k) * R + k;
#pragma unroll
            for (int r = 0; r < R; ++r) buf[(base + r * Ns) * TI + t] = v[m][r];
        }
    }
    __syncthreads();
}

template <int LOGN, int TI, int S>
__device__ __forceinline__ void fft_lines(float2 *buf, const float2 *tw) {
    constexpr int N = 1 << LOGN;
    constexpr int N8 = LOGN / 3, REM = LOGN % 3;
    int Ns = 1;
#pragma unroll
    for (int s = 0; s < N8; ++s) {
        stage<N, TI, 8, S>(buf, tw, Ns);
        Ns *= 8;
    }
    if constexpr (REM == 2) stage<N, TI, 4, S>(buf, tw, Ns);
    if constexpr (REM == 1) stage<N, TI, 2, S>(buf, tw, Ns);
}

struct AxisArgs {
    int64_t nlines;  // outer * inner
    int64_t inner;
    int Lin, Lout;   // line lengths in and out (one of them is N = 2^LOGN)
    int M, hM;       // kept modes along this axis and M/2
    const float *dec;
};

__device__ __forceinline__ int64_t line_base(int64_t line, int64_t inner, int L) {
    return (line / inner) * (int64_t)L * inner + line % inner;
}

// PRUNE_OUT: full n-point lines in, M modes out (type 1).
// otherwise: M modes in (zero elsewhere), full n-point lines out (type 2).
template <int LOGN, int TI, int S, bool PRUNE_OUT>
__global__ __launch_bounds__(FP_THREADS) void k_fft_axis(const float2 *__restrict__ in,
                                                         float2 *__restrict__ out, AxisArgs a) {
    constexpr int N = 1 << LOGN;
    __shared__ float2 buf[N * TI];
    __shared__ float2 tw[N];
    __shared__ int64_t lbi[TI], lbo[TI];  // line bases in and out (-1: past the end)
    const int tid = threadIdx.x;
    const int64_t ntile = (a.nlines + TI - 1) / TI;
    const int64_t line0 = xcd_remap(blockIdx.x, ntile) * TI;
    for (int m = tid; m < N; m += FP_THREADS) {
        double sn, cs;
        sincospi(2.0 * (double)m / (double)N, &sn, &cs);
        tw[m] = make_float2((float)cs, (float)(S * sn));
    }
    if (tid < TI) {
        const int64_t line = line0 + tid;
        const bool ok = line < a.nlines;
        lbi[tid] = ok ? line_base(line, a.inner, a.Lin) : -1;
        lbo[tid] = ok ? line_base(line, a.inner, a.Lout) : -1;
    }
    const bool contig = a.inner == 1;  // the lines are contiguous rows
    if constexpr (!PRUNE_OUT)
        for (int idx = tid; idx < N * TI; idx += FP_THREADS) buf[idx] = make_float2(0.f, 0.f);
    __syncthreads();
    if constexpr (PRUNE_OUT) {
#pragma unroll 8
        for (int idx = tid; idx < N * TI; idx += FP_THREADS) {
            const int t = contig ? idx / N : idx % TI, l = contig ? idx % N : idx / TI;
            const int64_t b = lbi[t];
            buf[l * TI + t] = b >= 0 ? in[b + (int64_t)l * a.inner] : make_float2(0.f, 0.f);
        }
    } else {
        const int nin = a.M * TI;
#pragma unroll 4
        for (int idx = tid; idx < nin; idx += FP_THREADS) {
            const int t = contig ? idx / a.M : idx % TI, i = contig ? idx % a.M : idx / TI;
            const int64_t b = lbi[t];
            if (b >= 0) {
                const float2 v = in[b + (int64_t)i * a.inner];
                const float d = a.dec[i];
                const int p = (i - a.hM + N) & (N - 1);
                buf[p * TI + t] = make_float2(v.x * d, v.y * d);
            }
        }
    }
    __syncthreads();
    fft_lines<LOGN, TI, S>(buf, tw);
    if constexpr (PRUNE_OUT) {
        const int nout = a.M * TI;
#pragma unroll 4
        for (int idx = tid; idx < nout; idx += FP_THREADS) {
            const int t = contig ? idx / a.M : idx % TI, i = contig ? idx % a.M : idx / TI;
            const int64_t b = lbo[t];
            if (b >= 0) {
                const int p = (i - a.hM + N) & (N - 1);
                const float2 v = buf[p * TI + t];
                const float d = a.dec[i];
                out[b + (int64_t)i * a.inner] = make_float2(v.x * d, v.y * d);
            }
        }
    } else {
#pragma unroll 8
        for (int idx = tid; idx < N * TI; idx += FP_THREADS) {
            const int t = contig ? idx / N : idx % TI, l = contig ? idx % N : idx / TI;
            const int64_t b = lbo[t];
            if (b >= 0) out[b + (int64_t)l * a.inner] = buf[l * TI + t];
        }
    }
}

constexpr int fp_ti(int logn) {
    return (FP_ELEMS >> logn) < 16 ? (FP_ELEMS >> logn) : 16;
}

template <int LOGN>
int launch_axis(bool prune_out, int isign, const float2 *in, float2 *out, const AxisArgs &a,
                hipStream_t s) {
    constexpr int TI = fp_ti(LOGN);
    const int64_t ntile = (a.nlines + TI - 1) / TI;
    if (ntile > 0x7fffffff) {
        set_error("fft: too many lines");
        return MN_EINVAL;
    }
    const dim3 grid((unsigned)ntile);
    if (prune_out) {
        if (isign > 0) k_fft_axis<LOGN, TI, 1, true><<<grid, FP_THREADS, 0, s>>>(in, out, a);
        else k_fft_axis<LOGN, TI, -1, true><<<grid, FP_THREADS, 0, s>>>(in, out, a);
    } else {
        if (isign > 0) k_fft_axis<LOGN, TI, 1, false><<<grid, FP_THREADS, 0, s>>>(in, out, a);
        else k_fft_axis<LOGN, TI, -1, false><<<grid, FP_THREADS, 0, s>>>(in, out, a);
    }
    MN_LAUNCH_CHECK("fft axis");
    return MN_OK;
}

constexpr int kMinLog = 4, kMaxLog = 12;

int log2_exact(int64_t n) {
    if (n < 1 || (n & (n - 1))) return -1;
    int l = 0;
    while ((int64_t(1) << l) < n) ++l;
    return l;
}

int run_axis(int logn, bool prune_out, int isign, const float2 *in, float2 *out,
             const AxisArgs &a, hipStream_t s) {
    switch (logn) {
        case 4: return launch_axis<4>(prune_out, isign, in, out, a, s);
        case 5: return launch_axis<5>(prune_out, isign, in, out, a, s);
        case 6: return launch_axis<6>(prune_out, isign, in, out, a, s);
        case 7: return launch_axis<7>(prune_out, isign, in, out, a, s);
        case 8: return launch_axis<8>(prune_out, isign, in, out, a, s);
        case 9: return launch_axis<9>(prune_out, isign, in, out, a, s);
        case 10: return launch_axis<10>(prune_out, isign, in, out, a, s);
        case 11: return launch_axis<11>(prune_out, isign, in, out, a, s);
        case 12: return launch_axis<12>(prune_out, isign, in, out, a, s);
    }
    set_error("fft: unsupported length");
    return MN_EINVAL;
}

struct Plan3 {
    int dim;
    int64_t n[3], N[3];
};

int check_pruned(int dim, const int64_t n_up[3], const int64_t N[3], int64_t batch, Plan3 *p) {
    MN_REQUIRE(dim >= 1 && dim <= 3, "pruned fft: dim must be 1, 2 or 3");
    MN_REQUIRE(batch >= 1, "pruned fft: batch must be >= 1");
    p->dim = dim;
    for (int d = 0; d < dim; ++d) {
        const int l = log2_exact(n_up[d]);
        MN_REQUIRE(l >= kMinLog && l <= kMaxLog,
                   "pruned fft: fine-grid sizes must be powers of two in [16, 4096]");
        MN_REQUIRE(N[d] >= 1 && N[d] <= n_up[d], "pruned fft: mode count out of range");
        p->n[d] = n_up[d];
        p->N[d] = N[d];
    }
    return MN_OK;
}

// Bytes of the two intermediate buffers (largest first) of either pipeline.
void work_sizes(const Plan3 &p, int64_t batch, int64_t *wa, int64_t *wb) {
    *wa = *wb = 0;
    if (p.dim == 2) *wa = 8 * batch * p.n[0] * p.N[1];
    if (p.dim == 3) {
        *wa = 8 * batch * p.n[0] * p.n[1] * p.N[2];
        *wb = 8 * batch * p.n[0] * p.N[1] * p.N[2];
    }
}

}  // namespace
}  // namespace mn

using namespace mn;

extern "C" {

int mn_fftp_supported(int dim, const int64_t n_up[3]) {
    if (dim < 1 || dim > 3) return 0;
    for (int d = 0; d < dim; ++d) {
        const int l = log2_exact(n_up[d]);
        if (l < kMinLog || l > kMaxLog) return 0;
    }
    return 1;
}

int64_t mn_fftp_work_bytes(int dim, const int64_t n_up[3], const int64_t N[3], int64_t batch) {
    Plan3 p{};
    if (check_pruned(dim, n_up, N, batch, &p)) return -1;
    int64_t wa, wb;
    work_sizes(p, batch, &wa, &wb);
    return wa + wb;
}

int mn_fft_crop_deconv(int dim, const int64_t n_up[3], const int64_t N[3], int64_t batch,
                       int isign, const void *grid, const float *const dec[3], void *work,
                       int64_t work_bytes, void *fk, mn_stream_t stream) {
    clear_error();
    Plan3 p{};
    int rc = check_pruned(dim, n_up, N, batch, &p);
    if (rc) return rc;
    int64_t wa, wb;
    work_sizes(p, batch, &wa, &wb);
    MN_REQUIRE(grid && fk && (wa + wb == 0 || work), "pruned fft: NULL pointer");
    MN_REQUIRE(work_bytes >= wa + wb, "pruned fft: work buffer too small");
    for (int d = 0; d < dim; ++d) MN_REQUIRE(dec[d], "pruned fft: NULL deconvolution vector");
    hipStream_t s = as_stream(stream);
    char *wbase = static_cast<char *>(work);
    float2 *bufs[2] = {reinterpret_cast<float2 *>(wbase), reinterpret_cast<float2 *>(wbase + wa)};
    const float2 *src = static_cast<const float2 *>(grid);
    int nb = 0;
    for (int d = dim - 1; d >= 0; --d) {
        AxisArgs a{};
        int64_t outer = batch, inner = 1;
        for (int e = 0; e < d; ++e) outer *= p.n[e];
        for (int e = d + 1; e < dim; ++e) inner *= p.N[e];
        a.nlines = outer * inner;
        a.inner = inner;
        a.Lin = (int)p.n[d];
        a.Lout = (int)p.N[d];
        a.M = (int)p.N[d];
        a.hM = (int)(p.N[d] / 2);
        a.dec = dec[d];
        float2 *dst = d == 0 ? static_cast<float2 *>(fk) : bufs[nb++];
        rc = run_axis(log2_exact(p.n[d]), true, isign, src, dst, a, s);
        if (rc) return rc;
        src = dst;
    }
    return MN_OK;
}

int mn_pad_deconv_fft(int dim, const int64_t n_up[3], const int64_t N[3], int64_t batch,
                      int isign, const void *fk, const float *const dec[3], void *work,
                      int64_t work_bytes, void *grid, mn_stream_t stream) {
    clear_error();
    Plan3 p{};
    int rc = check_pruned(dim, n_up, N, batch, &p);
    if (rc) return rc;
    int64_t wa, wb;
    work_sizes(p, batch, &wa, &wb);
    MN_REQUIRE(grid && fk && (wa + wb == 0 || work), "pruned fft: NULL pointer");
    MN_REQUIRE(work_bytes >= wa + wb, "pruned fft: work buffer too small");
    for (int d = 0; d < dim; ++d) MN_REQUIRE(dec[d], "pruned fft: NULL deconvolution vector");
    hipStream_t s = as_stream(stream);
    char *wbase = static_cast<char *>(work);
    // 3D: fk -> B (n0 N1 N2) -> A (n0 n1 N2) -> grid; 2D: fk -> A (n0 N1) -> grid
    float2 *A = reinterpret_cast<float2 *>(wbase), *B = reinterpret_cast<float2 *>(wbase + wa);
    const float2 *src = static_cast<const float2 *>(fk);
    for (int d = 0; d < dim; ++d) {
        AxisArgs a{};
        int64_t outer = batch, inner = 1;
        for (int e = 0; e < d; ++e) outer *= p.n[e];
        for (int e = d + 1; e < dim; ++e) inner *= p.N[e];
        a.nlines = outer * inner;
        a.inner = inner;
        a.Lin = (int)p.N[d];
        a.Lout = (int)p.n[d];
        a.M = (int)p.N[d];
        a.hM = (int)(p.N[d] / 2);
        a.dec = dec[d];
        float2 *dst;
        if (d == dim - 1) dst = static_cast<float2 *>(grid);
        else if (dim == 3 && d == 0) dst = B;
        else dst = A;
        rc = run_axis(log2_exact(p.n[d]), false, isign, src, dst, a, s);
        if (rc) return rc;
        src = dst;
    }
    return MN_OK;
}

}  // extern "C"
