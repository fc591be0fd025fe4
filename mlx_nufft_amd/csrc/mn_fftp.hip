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

#include <stdlib.h>

namespace mn {
namespace {

typedef float fp2 __attribute__((ext_vector_type(2)));
constexpr int FP_THREADS = 512;  // threads per workgroup (see fp_ti_shift)
constexpr int FP_ELEMS = 8192;  // complex values per workgroup tile (64 KB)

__device__ __forceinline__ float2 cadd(float2 a, float2 b) { return make_float2(a.x + b.x, a.y + b.y); }
__device__ __forceinline__ float2 csub(float2 a, float2 b) { return make_float2(a.x - b.x, a.y - b.y); }
__device__ __forceinline__ float2 cmul(float2 a, float2 b) {
    return make_float2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}
// out[i] = v; a streaming store when the lines are contiguous (the last
// axis: whole 64-byte runs per lane group, measured 1-2 % faster per
// transform), a plain one when they are strided (a streaming store of a
// partial line there doubled the type-2 passes' time)
__device__ __forceinline__ void store_out(float2 *out, int64_t i, float2 v, bool contig) {
    if (contig) {
        const fp2 val = {v.x, v.y};
        __builtin_nontemporal_store(val, reinterpret_cast<fp2 *>(out + i));
    } else {
        out[i] = v;
    }
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

// LDS slot of element l of line t in a tile of TI lines: rows of TI values,
// the column XOR-swizzled by the row so that both access patterns -- TI
// lines side by side (t fastest) and one line walked along l (l fastest) --
// spread over the LDS banks.
template <int TI>
__device__ __forceinline__ int lds_at(int l, int t) {
    constexpr int SH = TI >= 16 ? 0 : (TI >= 8 ? 1 : (TI >= 4 ? 2 : (TI >= 2 ? 3 : 4)));
    return l * TI + (t ^ ((l >> SH) & (TI - 1)));
}

// Butterfly b of a stage with NJ butterflies per line: (line t, index j).
// Contiguous lines put j fastest across lanes, strided ones t fastest, so
// that the global accesses of the first and last stages coalesce.
template <int TI, int NJ>
__device__ __forceinline__ void bfly_of(int b, bool contig, int &t, int &j) {
    if (contig) {
        t = b / NJ;
        j = b % NJ;
    } else {
        t = b % TI;
        j = b / TI;
    }
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

// Mode index i in [0, M) of FFT position p, or -1 if p is not kept.
template <int N>
__device__ __forceinline__ int mode_of(int p, int M, int hM) {
    if (p < M - hM) return p + hM;
    if (p >= N - hM) return p - (N - hM);
    return -1;
}

// Middle Stockham stage of radix R (LDS to LDS); Ns = product of the radices
// of the earlier stages; tw[m] = exp(S 2 pi i m / N).
template <int N, int TI, int R, int S>
__device__ __forceinline__ void stage(float2 *buf, const float2 *tw, int Ns) {
    constexpr int NJ = N / R, NB = NJ * TI;
    constexpr int MB = (NB + FP_THREADS - 1) / FP_THREADS;
    float2 v[MB][R];
    const int tstep = N / (Ns * R);
#pragma unroll
    for (int m = 0; m < MB; ++m) {
        const int b = threadIdx.x + m * FP_THREADS;
        if (b < NB) {
            const int t = b % TI, j = b / TI, k = j & (Ns - 1);
#pragma unroll
            for (int r = 0; r < R; ++r) v[m][r] = buf[lds_at<TI>(j + r * NJ, t)];
#pragma unroll
            for (int r = 1; r < R; ++r) v[m][r] = cmul(v[m][r], tw[k * r * tstep]);
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
            for (int r = 0; r < R; ++r) buf[lds_at<TI>(base + r * Ns, t)] = v[m][r];
        }
    }
    __syncthreads();
}

// PRUNE_OUT: full n-point lines in, M modes out (type 1).
// otherwise: M modes in (zero elsewhere), full n-point lines out (type 2).
// The first radix-8 stage reads its inputs straight from global memory and
// the last stage writes its outputs straight back; LDS carries the stages
// in between.
template <int LOGN, int TI, int S, bool PRUNE_OUT>
__global__ __launch_bounds__(FP_THREADS) void k_fft_axis(const float2 *__restrict__ in,
                                                         float2 *__restrict__ out, AxisArgs a) {
    constexpr int N = 1 << LOGN;
    constexpr int N8 = LOGN / 3, REM = LOGN % 3;
    constexpr int RL = REM == 0 ? 8 : (REM == 1 ? 2 : 4);  // radix of the last stage
    static_assert(LOGN >= 4, "n >= 16");
    __shared__ float2 buf[N * TI];
    __shared__ float2 tw[N];
    __shared__ int64_t lbi[TI], lbo[TI];  // line bases in and out (-1: past the end)
    const int tid = threadIdx.x;
    const int64_t ntile = (a.nlines + TI - 1) / TI;
    const int64_t line0 = xcd_remap(blockIdx.x, ntile) * TI;
    const bool contig = a.inner == 1;  // the lines are contiguous rows
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
    __syncthreads();

    // ---- first stage: radix 8, Ns = 1, inputs from global memory ----
    {
        constexpr int NJ = N / 8, NB = NJ * TI, MB = (NB + FP_THREADS - 1) / FP_THREADS;
        float2 v[MB][8];
#pragma unroll
        for (int m = 0; m < MB; ++m) {
            const int b = tid + m * FP_THREADS;
            int t = 0, j = 0;
            bfly_of<TI, NJ>(b, contig, t, j);
            const int64_t lb = b < NB ? lbi[t] : -1;
            if constexpr (PRUNE_OUT) {
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    const int p = j + r * NJ;
                    v[m][r] = lb >= 0 ? in[lb + (int64_t)p * a.inner] : make_float2(0.f, 0.f);
                }
            } else {
                // every mode and factor load is issued (at index 0 where no
                // mode is kept) before any is used: loaded and scaled inside
                // a branch, each waited for its own pair of loads
                float2 y[8];
                float d[8];
                bool ok[8];
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    const int i = mode_of<N>(j + r * NJ, a.M, a.hM);
                    ok[r] = lb >= 0 && i >= 0;
                    y[r] = in[ok[r] ? lb + (int64_t)i * a.inner : 0];
                    d[r] = a.dec[ok[r] ? i : 0];
                }
#pragma unroll
                for (int r = 0; r < 8; ++r)
                    v[m][r] = ok[r] ? make_float2(y[r].x * d[r], y[r].y * d[r])
                                    : make_float2(0.f, 0.f);
            }
        }
#pragma unroll
        for (int m = 0; m < MB; ++m) {
            const int b = tid + m * FP_THREADS;
            if (b < NB) {
                int t, j;
                bfly_of<TI, NJ>(b, contig, t, j);
                dft8<S>(v[m]);
#pragma unroll
                for (int r = 0; r < 8; ++r) buf[lds_at<TI>(j * 8 + r, t)] = v[m][r];
            }
        }
        __syncthreads();
    }

    // ---- middle stages ----
    int Ns = 8;
#pragma unroll
    for (int s = 1; s < (REM == 0 ? N8 - 1 : N8); ++s) {
        stage<N, TI, 8, S>(buf, tw, Ns);
        Ns *= 8;
    }

    // ---- last stage: radix RL, Ns = N / RL, outputs to global memory ----
    {
        constexpr int NJ = N / RL, NB = NJ * TI, MB = (NB + FP_THREADS - 1) / FP_THREADS;
#pragma unroll
        for (int m = 0; m < MB; ++m) {
            const int b = tid + m * FP_THREADS;
            if (b < NB) {
                int t, j;
                bfly_of<TI, NJ>(b, contig, t, j);
                // the kept modes' deconvolution factors are loaded first, all
                // at once, under the LDS reads and the DFT (loaded at the
                // store, each waited for its own)
                int im[RL];
                float dm[RL];
                if constexpr (PRUNE_OUT) {
#pragma unroll
                    for (int r = 0; r < RL; ++r) {
                        im[r] = mode_of<N>(j + r * NJ, a.M, a.hM);
                        dm[r] = a.dec[im[r] >= 0 ? im[r] : 0];
                    }
                }
                float2 v[RL];
#pragma unroll
                for (int r = 0; r < RL; ++r) v[r] = buf[lds_at<TI>(j + r * NJ, t)];
#pragma unroll
                for (int r = 1; r < RL; ++r) v[r] = cmul(v[r], tw[j * r]);
                dft<RL, S>(v);
                const int64_t lb = lbo[t];
                if (lb >= 0) {
#pragma unroll
                    for (int r = 0; r < RL; ++r) {
                        const int p = j + r * NJ;  // natural-order output position
                        if constexpr (PRUNE_OUT) {
                            if (im[r] >= 0)
                                store_out(out, lb + (int64_t)im[r] * a.inner,
                                          make_float2(v[r].x * dm[r], v[r].y * dm[r]), contig);
                        } else {
                            store_out(out, lb + (int64_t)p * a.inner, v[r], contig);
                        }
                    }
                }
            }
        }
    }
}

constexpr int fp_ti(int logn) {
    return (FP_ELEMS >> logn) < 16 ? (FP_ELEMS >> logn) : 16;
}

template <int LOGN, int TI>
int launch_axis_ti(bool prune_out, int isign, const float2 *in, float2 *out, const AxisArgs &a,
                   hipStream_t s) {
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

// Lines per workgroup: fp_ti(LOGN) fills 64 KB of LDS; half of that, with
// 512 threads, runs fastest on MI355X. At 512^3 the type-1 passes (crop)
// took 0.556 ms, against 0.587 with 256 threads, a quarter tile for the
// contiguous lines and half for the strided ones (0.588 with all 16 lines
// on the strided ones), and the type-2 passes (pad) 0.627 ms against 0.711
// with 256 threads and quarter tiles; a quarter tile at 512 threads took
// 0.59 and 0.74 ms, an eighth 0.72 and 0.97. The 2D batched passes of
// 2048^2 x 8: 0.208 against 0.22 ms. More resident waves per CU keep more
// loads in flight.
// MN_FFT_TI_SHIFT / MN_FFT_TI_SHIFT_STRIDED override the shifts (tuning).
int fp_ti_shift(bool contig) {
    static const int vc = [] {
        const char *e = getenv("MN_FFT_TI_SHIFT");
        return e ? atoi(e) : 1;
    }();
    static const int vs = [] {
        const char *e = getenv("MN_FFT_TI_SHIFT_STRIDED");
        return e ? atoi(e) : -1;
    }();
    if (contig) return vc;
    return vs >= 0 ? vs : 1;
}

template <int LOGN>
int launch_axis(bool prune_out, int isign, const float2 *in, float2 *out, const AxisArgs &a,
                hipStream_t s) {
    constexpr int TI = fp_ti(LOGN);
    const int shift = fp_ti_shift(a.inner == 1);
    if constexpr (TI >= 8) {
        if (shift >= 3) return launch_axis_ti<LOGN, TI / 8>(prune_out, isign, in, out, a, s);
    }
    if constexpr (TI >= 4) {
        if (shift == 2) return launch_axis_ti<LOGN, TI / 4>(prune_out, isign, in, out, a, s);
    }
    if constexpr (TI >= 2) {
        if (shift == 1) return launch_axis_ti<LOGN, TI / 2>(prune_out, isign, in, out, a, s);
    }
    return launch_axis_ti<LOGN, TI>(prune_out, isign, in, out, a, s);
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
