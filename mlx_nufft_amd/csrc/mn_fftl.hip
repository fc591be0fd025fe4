// Batched zero-padding line FFTs in double precision, for the type-3 inner
// grid.
//
// The type-3 inner grid is the deconvolved spread grid (nf_d values per
// axis) zero-padded to n_up_d and transformed in all three axes. Instead of
// a pad kernel and a full 3D transform over the padded grid, one pass per
// axis transforms only the lines that can be non-zero and fuses that axis's
// deconvolution and zero padding into the line load:
//
//   bf (nf0 nf1 nf2) -z-> (nf0 nf1 n2) -y-> (nf0 n1 n2) -x-> H (n0 n1 n2)
//
// Each pass reads an array of shape (A, nin, B) and writes (A, n, B): line
// (a, b) is in[a, :, b]; its element m (times dec[m]) sits at FFT index
// (m - nin/2) mod n with zeros elsewhere, and out[a, r, b] is the
// unnormalised sum over that line of x[p] exp(isign 2 pi i p r / n). The last
// pass can round straight to complex64.
//
// One workgroup holds TI whole lines in LDS (n <= 8192, so a line of 7200
// doubles fits where the runtime's transform splits it into several passes)
// and runs mixed-radix Stockham stages of radix 8, 4, 2, 3 and 5 over them;
// each stage reads its butterflies into registers, waits at a barrier and
// writes them back in place. The twiddle exp(isign 2 pi i m / n) for each
// butterfly comes from a per-(device, n, sign) table computed once with fp64
// sincospi; its powers are formed by complex multiplication. TI consecutive
// lines share a tile, so a strided axis (B > 1) reads TI contiguous values
// per element and the contiguous axis (B == 1) reads whole runs of lines.
// Workgroups are remapped so consecutive tiles share an XCD (and its L2)
// when a tile covers less than a cache line.
//
// ref: gpu_t3.py:630-651 (t3pad: pad + mode deconvolution), gpu_t3.py:94-148
// (fft_axis), gpu_t3.py:697-741 (t3padz: the slab path's fused pad, deconv
// and z-DFT, which this generalises to every axis).
#include "mn_common.h"

#include <algorithm>
#include <map>
#include <mutex>
#include <tuple>

namespace mn {
namespace {

constexpr int FL_NMAX = 8192;   // longest line: 128 KB of LDS
constexpr int FL_WIDE = 5120;   // values of an unpadded strided tile (80 KB)
constexpr int FL_MAXST = 16;

// ti = 2^lti lines per tile, stored element-major in LDS (value p of line l
// at p*ts + l, ts = ti + 1 for ti > 1 so that radix strides do not map the
// lanes of a wave onto the same banks; ts = ti for the unpadded tiles of
// 8 or more lines, see mn_fft64_lines).
struct FlPlan {
    int n, nin, lti, ts, nst;
    float rn, rnin;           // 1/n, 1/nin
    int rad[FL_MAXST];
    int ns[FL_MAXST];         // product of the radices before stage s
    float rns[FL_MAXST];      // 1/ns[s]
};

// q = x / d for 0 <= x < 2^20 and d >= 1, from a float reciprocal r ~ 1/d:
// the estimate is off by at most one, fixed by one comparison each way.
__device__ __forceinline__ int fdiv(int x, int d, float r) {
    int q = (int)((float)x * r);
    const int rem = x - q * d;
    q += (rem >= d) - (rem < 0);
    return q;
}

__device__ __forceinline__ double2 dadd(double2 a, double2 b) { return make_double2(a.x + b.x, a.y + b.y); }
__device__ __forceinline__ double2 dsub(double2 a, double2 b) { return make_double2(a.x - b.x, a.y - b.y); }
__device__ __forceinline__ double2 dmul(double2 a, double2 b) {
    return make_double2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}
__device__ __forceinline__ double2 dscale(double2 a, double s) { return make_double2(a.x * s, a.y * s); }
// a * (S i)
template <int S>
__device__ __forceinline__ double2 dmul_si(double2 a) {
    return S > 0 ? make_double2(-a.y, a.x) : make_double2(a.y, -a.x);
}

// In-register DFTs X[k] = sum_m v[m] exp(S 2 pi i m k / R).
template <int S>
__device__ __forceinline__ void ddft2(double2 *v) {
    const double2 a = v[0];
    v[0] = dadd(a, v[1]);
    v[1] = dsub(a, v[1]);
}

template <int S>
__device__ __forceinline__ void ddft4(double2 &v0, double2 &v1, double2 &v2, double2 &v3) {
    const double2 a0 = dadd(v0, v2), a1 = dsub(v0, v2), a2 = dadd(v1, v3);
    const double2 a3 = dmul_si<S>(dsub(v1, v3));
    v0 = dadd(a0, a2);
    v2 = dsub(a0, a2);
    v1 = dadd(a1, a3);
    v3 = dsub(a1, a3);
}

template <int S>
__device__ __forceinline__ void ddft4(double2 *v) { ddft4<S>(v[0], v[1], v[2], v[3]); }

template <int S>
__device__ __forceinline__ void ddft8(double2 *v) {
    constexpr double R2 = 0.70710678118654752440;  // sqrt(1/2)
    double2 e0 = v[0], e1 = v[2], e2 = v[4], e3 = v[6];
    double2 o0 = v[1], o1 = v[3], o2 = v[5], o3 = v[7];
    ddft4<S>(e0, e1, e2, e3);
    ddft4<S>(o0, o1, o2, o3);
    // o_k *= exp(S i pi k / 4)
    o1 = make_double2((o1.x - S * o1.y) * R2, (o1.y + S * o1.x) * R2);
    o2 = dmul_si<S>(o2);
    o3 = make_double2((-o3.x - S * o3.y) * R2, (-o3.y + S * o3.x) * R2);
    v[0] = dadd(e0, o0);
    v[4] = dsub(e0, o0);
    v[1] = dadd(e1, o1);
    v[5] = dsub(e1, o1);
    v[2] = dadd(e2, o2);
    v[6] = dsub(e2, o2);
    v[3] = dadd(e3, o3);
    v[7] = dsub(e3, o3);
}

// Radix 3: w = exp(S 2 pi i / 3) = -1/2 + S i sqrt(3)/2.
template <int S>
__device__ __forceinline__ void ddft3(double2 *v) {
    constexpr double H3 = 0.86602540378443864676;  // sqrt(3)/2
    const double2 t1 = dadd(v[1], v[2]);
    const double2 t2 = dsub(v[0], dscale(t1, 0.5));
    const double2 t3 = dscale(dmul_si<S>(dsub(v[1], v[2])), H3);
    v[0] = dadd(v[0], t1);
    v[1] = dadd(t2, t3);
    v[2] = dsub(t2, t3);
}

// Radix 5 with c_k = cos(2 pi k / 5), s_k = sin(2 pi k / 5):
//   X1,4 = v0 + c1 a1 + c2 a2 +- S i (s1 b1 + s2 b2)
//   X2,3 = v0 + c2 a1 + c1 a2 +- S i (s2 b1 - s1 b2)
// with a1 = v1 + v4, b1 = v1 - v4, a2 = v2 + v3, b2 = v2 - v3.
template <int S>
__device__ __forceinline__ void ddft5(double2 *v) {
    constexpr double C1 = 0.30901699437494742410, C2 = -0.80901699437494742410;
    constexpr double S1 = 0.95105651629515357212, S2 = 0.58778525229247312917;
    const double2 a1 = dadd(v[1], v[4]), b1 = dsub(v[1], v[4]);
    const double2 a2 = dadd(v[2], v[3]), b2 = dsub(v[2], v[3]);
    const double2 v0 = v[0];
    const double2 p1 = dadd(v0, dadd(dscale(a1, C1), dscale(a2, C2)));
    const double2 p2 = dadd(v0, dadd(dscale(a1, C2), dscale(a2, C1)));
    const double2 q1 = dmul_si<S>(dadd(dscale(b1, S1), dscale(b2, S2)));
    const double2 q2 = dmul_si<S>(dsub(dscale(b1, S2), dscale(b2, S1)));
    v[0] = dadd(v0, dadd(a1, a2));
    v[1] = dadd(p1, q1);
    v[4] = dsub(p1, q1);
    v[2] = dadd(p2, q2);
    v[3] = dsub(p2, q2);
}

template <int S, int R>
__device__ __forceinline__ void ddft(double2 *v) {
    if constexpr (R == 2) ddft2<S>(v);
    else if constexpr (R == 3) ddft3<S>(v);
    else if constexpr (R == 4) ddft4<S>(v);
    else if constexpr (R == 5) ddft5<S>(v);
    else ddft8<S>(v);
}

// One Stockham stage of radix R over the ti lines of n values in LDS,
// after stages whose radices multiply to Ns: butterfly j of a line takes
// x[j + r n/R] times w^r (w = exp(S 2 pi i k / (Ns R)), k = j mod Ns), runs
// a radix-R DFT and stores output r at (j / Ns) Ns R + k + r Ns. Butterfly
// b of the tile is (line b mod ti, j = b / ti), so neighbouring lanes touch
// neighbouring LDS words. Every butterfly of the stage is read into
// registers before the barrier and written back after it.
template <int S, int R, int T, int VALS>
__device__ __forceinline__ void fl_stage(double2 *buf, const double2 *__restrict__ tw, int n,
                                         int lti, int ts, int Ns, float rNs, int tid) {
    constexpr int F = (VALS / R + T - 1) / T;
    const int nr = n / R;
    const int nbf = nr << lti;
    const int tws = n / (Ns * R);
    const int lmask = (1 << lti) - 1;
    double2 v[F][R];
#pragma unroll
    for (int f = 0; f < F; ++f) {
        const int b = tid + f * T;
        if (b < nbf) {
            const int l = b & lmask, j = b >> lti;
            const int k = j - fdiv(j, Ns, rNs) * Ns;
            const double2 *src = buf + j * ts + l;
            v[f][0] = src[0];
            const double2 w = tw[k * tws];
            double2 wr = w;
#pragma unroll
            for (int r = 1; r < R; ++r) {
                v[f][r] = dmul(src[r * nr * ts], wr);
                if (r + 1 < R) wr = dmul(wr, w);
            }
            ddft<S, R>(v[f]);
        }
    }
    __syncthreads();
#pragma unroll
    for (int f = 0; f < F; ++f) {
        const int b = tid + f * T;
        if (b < nbf) {
            const int l = b & lmask, j = b >> lti;
            const int k = j - fdiv(j, Ns, rNs) * Ns;
            double2 *dst = buf + ((j - k) * R + k) * ts + l;
#pragma unroll
            for (int r = 0; r < R; ++r) dst[r * Ns * ts] = v[f][r];
        }
    }
    __syncthreads();
}

// T threads, at most VALS values (ti * n) per tile. With B == 1 the tile's
// lines are consecutive runs of the input and output; with B > 1, ti divides
// B, so the tile's lines share a and element m of all of them is ti
// contiguous values.
template <int S, bool C64OUT, int T, int VALS>
__global__ __launch_bounds__(T) void k_fft64_lines(const double2 *__restrict__ in,
                                                   void *__restrict__ out,
                                                   const double *__restrict__ dec,
                                                   const double2 *__restrict__ tw, int nlines,
                                                   int Bn, int Bo, int ntiles, FlPlan p) {
    extern __shared__ double2 fl_buf[];
    const int n = p.n, nin = p.nin, lti = p.lti, ts = p.ts, tid = threadIdx.x;
    const int ti = 1 << lti, lmask = ti - 1;
    const int li0 = (int)xcd_remap(blockIdx.x, ntiles) << lti;
    const int half = nin / 2;
    // the zero padding: FFT indices [nin - half, n - half) of every line
    const int gap0 = nin - half;
    for (int e = tid; e < (n - nin) << lti; e += T)
        fl_buf[(gap0 + (e >> lti)) * ts + (e & lmask)] = make_double2(0.0, 0.0);
    // All of a thread's loads (at most FV values and their dec factors) are
    // issued before the first LDS write, at clamped (in-range) indices, so
    // that they are in flight together; a load-then-store loop kept one
    // load per thread in flight.
    constexpr int FV = (VALS + T - 1) / T;
    double2 fv[FV];
    double fd[FV];
    if (Bn == 1) {
        const int64_t base = (int64_t)li0 * nin;
        const int cnt = min(ti, nlines - li0) * nin;
#pragma unroll
        for (int i = 0; i < FV; ++i) {
            const int e = min(tid + i * T, cnt - 1);
            fv[i] = in[base + e];
            fd[i] = dec ? dec[e - fdiv(e, nin, p.rnin) * nin] : 1.0;
        }
#pragma unroll
        for (int i = 0; i < FV; ++i) {
            const int e = tid + i * T;
            if (e < cnt) {
                const int l = fdiv(e, nin, p.rnin), m = e - l * nin;
                const double2 v = dec ? dscale(fv[i], fd[i]) : fv[i];
                const int r = m < half ? m - half + n : m - half;
                fl_buf[r * ts + l] = v;
            }
        }
    } else {
        const int a = li0 / Bn, b0 = li0 - a * Bn;
        const double2 *src = in + (int64_t)a * nin * Bn + b0;
        const int cnt = nin << lti;
#pragma unroll
        for (int i = 0; i < FV; ++i) {
            const int e = min(tid + i * T, cnt - 1);
            fv[i] = src[(int64_t)(e >> lti) * Bn + (e & lmask)];
            fd[i] = dec ? dec[e >> lti] : 1.0;
        }
#pragma unroll
        for (int i = 0; i < FV; ++i) {
            const int e = tid + i * T;
            if (e < cnt) {
                const int m = e >> lti, l = e & lmask;
                const double2 v = dec ? dscale(fv[i], fd[i]) : fv[i];
                const int r = m < half ? m - half + n : m - half;
                fl_buf[r * ts + l] = v;
            }
        }
    }
    __syncthreads();
    for (int s = 0; s < p.nst; ++s) {
        const int Ns = p.ns[s];
        const float rNs = p.rns[s];
        switch (p.rad[s]) {
            case 8: fl_stage<S, 8, T, VALS>(fl_buf, tw, n, lti, ts, Ns, rNs, tid); break;
            case 4: fl_stage<S, 4, T, VALS>(fl_buf, tw, n, lti, ts, Ns, rNs, tid); break;
            case 2: fl_stage<S, 2, T, VALS>(fl_buf, tw, n, lti, ts, Ns, rNs, tid); break;
            case 3: fl_stage<S, 3, T, VALS>(fl_buf, tw, n, lti, ts, Ns, rNs, tid); break;
            default: fl_stage<S, 5, T, VALS>(fl_buf, tw, n, lti, ts, Ns, rNs, tid); break;
        }
    }
    auto put = [&](int64_t o, double2 v) {
        if constexpr (C64OUT)
            reinterpret_cast<float2 *>(out)[o] = make_float2((float)v.x, (float)v.y);
        else
            reinterpret_cast<double2 *>(out)[o] = v;
    };
    if (Bo == 1) {
        const int64_t base = (int64_t)li0 * n;
        const int cnt = min(ti, nlines - li0) * n;
        for (int e = tid; e < cnt; e += T) {
            const int l = fdiv(e, n, p.rn), r = e - l * n;
            put(base + e, fl_buf[r * ts + l]);
        }
    } else {
        const int a = li0 / Bo, b0 = li0 - a * Bo;
        const int64_t base = (int64_t)a * n * Bo + b0;
        const int cnt = min(ti, nlines - li0);
        for (int e = tid; e < n << lti; e += T) {
            const int r = e >> lti, l = e & lmask;
            if (l < cnt) put(base + (int64_t)r * Bo + l, fl_buf[r * ts + l]);
        }
    }
}

// out[b][c][r] = in[b][r][c] for complex128 (Bt, R, C) -> (Bt, C, R), through
// 32 x 32 LDS tiles (one pad column keeps the column reads off one bank).
__global__ __launch_bounds__(256) void k_transpose_c128(const double2 *__restrict__ in,
                                                        double2 *__restrict__ out, int R, int C) {
    __shared__ double2 t[32][33];
    const int64_t plane = (int64_t)blockIdx.z * R * C;
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
#pragma unroll
    for (int k = 0; k < 32; k += 8) {
        const int r = r0 + ty + k, c = c0 + tx;
        if (r < R && c < C) t[ty + k][tx] = in[plane + (int64_t)r * C + c];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 32; k += 8) {
        const int c = c0 + ty + k, r = r0 + tx;
        if (r < R && c < C) out[plane + (int64_t)c * R + r] = t[tx][ty + k];
    }
}

// Long contiguous lines (n > 4096, B == 1, one line per tile): a persistent
// workgroup per CU walks lines gridDim.x apart. The next line's inputs are
// loaded into registers (up to 8 complex128 per thread) right after the
// current line is in LDS, so they arrive while its stages run, and the LDS
// fill of a line is register to LDS. One 7200-point fp64 line fills the
// LDS, so without this a CU loads, transforms and stores strictly in turn.
constexpr int FLL_THREADS = 1024;
constexpr int FLL_PT = FL_NMAX / FLL_THREADS;  // input values per thread

template <int S, bool C64OUT>
__global__ __launch_bounds__(FLL_THREADS) void k_fft64_long(const double2 *__restrict__ in,
                                                            void *__restrict__ out,
                                                            const double *__restrict__ dec,
                                                            const double2 *__restrict__ tw,
                                                            int nlines, FlPlan p) {
    extern __shared__ double2 fl_buf[];
    const int n = p.n, nin = p.nin, tid = threadIdx.x;
    const int half = nin / 2, gap0 = nin - half;
    double2 nxt[FLL_PT];
    auto load = [&](int line) {
        const double2 *src = in + (int64_t)line * nin;
#pragma unroll
        for (int i = 0; i < FLL_PT; ++i) {
            const int e = tid + i * FLL_THREADS;
            nxt[i] = e < nin ? src[e] : make_double2(0.0, 0.0);
        }
    };
    int line = blockIdx.x;
    if (line < nlines) load(line);
    for (; line < nlines; line += gridDim.x) {
        for (int e = tid; e < n - nin; e += FLL_THREADS) fl_buf[gap0 + e] = make_double2(0.0, 0.0);
#pragma unroll
        for (int i = 0; i < FLL_PT; ++i) {
            const int e = tid + i * FLL_THREADS;
            if (e < nin) {
                double2 v = nxt[i];
                if (dec) v = dscale(v, dec[e]);
                fl_buf[e < half ? e - half + n : e - half] = v;
            }
        }
        __syncthreads();
        const int nl = line + gridDim.x;
        if (nl < nlines) load(nl);
        for (int st = 0; st < p.nst; ++st) {
            const int Ns = p.ns[st];
            const float rNs = p.rns[st];
            switch (p.rad[st]) {
                case 8: fl_stage<S, 8, FLL_THREADS, FL_NMAX>(fl_buf, tw, n, 0, 1, Ns, rNs, tid); break;
                case 4: fl_stage<S, 4, FLL_THREADS, FL_NMAX>(fl_buf, tw, n, 0, 1, Ns, rNs, tid); break;
                case 2: fl_stage<S, 2, FLL_THREADS, FL_NMAX>(fl_buf, tw, n, 0, 1, Ns, rNs, tid); break;
                case 3: fl_stage<S, 3, FLL_THREADS, FL_NMAX>(fl_buf, tw, n, 0, 1, Ns, rNs, tid); break;
                default: fl_stage<S, 5, FLL_THREADS, FL_NMAX>(fl_buf, tw, n, 0, 1, Ns, rNs, tid); break;
            }
        }
        const int64_t base = (int64_t)line * n;
        for (int e = tid; e < n; e += FLL_THREADS) {
            const double2 v = fl_buf[e];
            if constexpr (C64OUT)
                reinterpret_cast<float2 *>(out)[base + e] = make_float2((float)v.x, (float)v.y);
            else
                reinterpret_cast<double2 *>(out)[base + e] = v;
        }
        __syncthreads();  // the stores have read fl_buf before the next fill
    }
}

// tw[m] = exp(S 2 pi i m / n)
__global__ void k_fl_twiddles(double2 *tw, int n, int S) {
    const int m = blockIdx.x * blockDim.x + threadIdx.x;
    if (m >= n) return;
    double s, c;
    sincospi(2.0 * (double)m / (double)n, &s, &c);
    tw[m] = make_double2(c, S * s);
}

// Radices for n = 2^a 3^b 5^c, largest stages first; 0 if n has another
// factor or needs more than FL_MAXST stages.
int fl_radices(int64_t n, int *rad) {
    int ns = 0;
    int64_t m = n;
    for (int R : {5, 3}) {
        while (m % R == 0) {
            if (ns == FL_MAXST) return 0;
            rad[ns++] = R;
            m /= R;
        }
    }
    for (int R : {8, 4, 2}) {
        while (m % R == 0) {
            if (ns == FL_MAXST) return 0;
            rad[ns++] = R;
            m /= R;
        }
    }
    return m == 1 ? ns : 0;
}

std::mutex g_tw_mu;
std::map<std::tuple<int, int, int>, double2 *> g_tw;

int twiddles(int n, int S, hipStream_t s, const double2 **out) {
    int dev = 0;
    MN_HIP_CHECK(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_tw_mu);
    const auto key = std::make_tuple(dev, n, S);
    auto it = g_tw.find(key);
    if (it == g_tw.end()) {
        double2 *t = nullptr;
        MN_HIP_CHECK(hipMalloc(&t, sizeof(double2) * (size_t)n));
        k_fl_twiddles<<<(n + 255) / 256, 256, 0, s>>>(t, n, S);
        MN_LAUNCH_CHECK("fft64 twiddles");
        // later calls may come on other streams: the table is complete first
        MN_HIP_CHECK(hipStreamSynchronize(s));
        it = g_tw.emplace(key, t).first;
    }
    *out = it->second;
    return MN_OK;
}

}  // namespace

void fftl_cache_clear() {
    std::lock_guard<std::mutex> lock(g_tw_mu);
    for (auto &kv : g_tw) (void)hipFree(kv.second);
    g_tw.clear();
}

}  // namespace mn

using namespace mn;

extern "C" {

int mn_fft64_lines_supported(int64_t n) {
    int rad[FL_MAXST];
    return n >= 2 && n <= FL_NMAX && fl_radices(n, rad) > 0;
}

int mn_fft64_lines(int64_t A, int64_t nin, int64_t B, int64_t n, int isign, const void *in,
                   const double *dec, void *out, int out_c64, int out_layout,
                   mn_stream_t stream) {
    clear_error();
    MN_REQUIRE(in && out, "fft64_lines: NULL input or output");
    MN_REQUIRE(out_layout >= 0 && out_layout <= 2, "fft64_lines: out_layout must be 0, 1 or 2");
    MN_REQUIRE(in != out, "fft64_lines: input and output must not alias");
    MN_REQUIRE(A >= 1 && B >= 1, "fft64_lines: A and B must be >= 1");
    MN_REQUIRE(mn_fft64_lines_supported(n), "fft64_lines: n must be 2^a 3^b 5^c in [2, 8192]");
    MN_REQUIRE(nin >= 1 && nin <= n, "fft64_lines: nin must be in [1, n]");
    MN_REQUIRE(B < (int64_t(1) << 31) && A * B < (int64_t(1) << 31),
               "fft64_lines: A*B (the line count) must be < 2^31");
    FlPlan p{};
    p.n = (int)n;
    p.nin = (int)nin;
    p.nst = fl_radices(n, p.rad);
    p.rn = 1.0f / (float)n;
    p.rnin = 1.0f / (float)nin;
    for (int s = 0, ns = 1; s < p.nst; ns *= p.rad[s], ++s) {
        p.ns[s] = ns;
        p.rns[s] = 1.0f / (float)ns;
    }
    const int nlines = (int)(A * B);
    // lines up to 4096 long: 512 threads and at most 4096 values (64 KB) per
    // tile, two tiles per CU; longer lines: one line, 1024 threads (the LDS
    // holds one such tile per CU, so its waves are all the latency hiding
    // there is). Measured on MI355X: 640^3 passes 5.70 ms with 512 threads,
    // 6.59 with 256, 7.8 with 1024; 7200-point lines of a 7200^2 x 24 grid
    // 11.3 ms with 1024 threads, 13.8 with 512.
    const bool longl = n > 4096;
    const int vals = longl ? 8192 : 4096;
    int lti = 0;
    // output line stride: B (layout 0), all lines when the line index runs
    // fastest (1), or 1 when each line's values are contiguous (2)
    const int64_t Bo = out_layout == 1 ? A * B : (out_layout == 2 ? 1 : B);
    int bpow = B > 1 ? __builtin_ctzll((unsigned long long)B) : 30;
    if (Bo > 1) bpow = min(bpow, (int)__builtin_ctzll((unsigned long long)Bo));
    while (lti < bpow && (int64_t)(1 << (lti + 1)) <= nlines &&
           n * ((1 << (lti + 1)) + 1) <= vals)
        ++lti;
    // A tile without the pad column, of up to FL_WIDE values (80 KB: two
    // workgroups still share a CU), is taken when it holds twice the lines,
    // and at least 8: strided lines (B > 1) then read 2 ti contiguous values
    // per element. A 16-lane LDS access of the stages spans at most two
    // butterflies, so their conflicts stay rare; the fill and drain of
    // contiguous lines, which walk one line per 16 lanes, conflict, and
    // still come out ahead. Measured on MI355X at 640^3 (type-3 Table I,
    // 8 lines per tile instead of 4 padded ones at three workgroups per
    // CU): the strided passes took the transform from 5.60 to 5.15 ms, the
    // contiguous z pass then from 5.12 to 5.01 ms.
    bool wide = false;
    if (!longl && lti >= 2 && lti < bpow && (int64_t(2) << lti) <= nlines &&
        n * (int64_t(2) << lti) <= FL_WIDE) {
        ++lti;
        wide = true;
    }
    p.lti = lti;
    p.ts = wide ? (1 << lti) : (lti > 0 ? (1 << lti) + 1 : 1);
    const int ntiles = (nlines + (1 << lti) - 1) >> lti;
    hipStream_t s = as_stream(stream);
    const int S = isign >= 0 ? 1 : -1;
    const double2 *tw = nullptr;
    int rc = twiddles((int)n, S, s, &tw);
    if (rc) return rc;
    const size_t lds = sizeof(double2) * (size_t)n * (size_t)p.ts;
    MN_REQUIRE(lds <= (size_t)max_lds_per_block(), "fft64_lines: line does not fit in LDS");
    if (longl && B == 1 && Bo == 1) {
        int dev = 0, ncu = 0;
        MN_HIP_CHECK(hipGetDevice(&dev));
        MN_HIP_CHECK(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev));
        const int nwg = (int)std::min<int64_t>(nlines, std::max(1, ncu));
        auto lk = S > 0 ? (out_c64 ? k_fft64_long<1, true> : k_fft64_long<1, false>)
                        : (out_c64 ? k_fft64_long<-1, true> : k_fft64_long<-1, false>);
        const size_t llds = sizeof(double2) * (size_t)n;
        if (llds > 65536)
            MN_HIP_CHECK(hipFuncSetAttribute((const void *)lk,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)llds));
        lk<<<(unsigned)nwg, FLL_THREADS, llds, s>>>(static_cast<const double2 *>(in), out, dec, tw,
                                                    nlines, p);
        MN_LAUNCH_CHECK("fft64_lines (long)");
        return MN_OK;
    }
    using K = void (*)(const double2 *, void *, const double *, const double2 *, int, int, int,
                       int, FlPlan);
    K kern;
    if (wide)
        kern = S > 0 ? (out_c64 ? k_fft64_lines<1, true, 512, FL_WIDE> : k_fft64_lines<1, false, 512, FL_WIDE>)
                     : (out_c64 ? k_fft64_lines<-1, true, 512, FL_WIDE> : k_fft64_lines<-1, false, 512, FL_WIDE>);
    else if (longl)
        kern = S > 0 ? (out_c64 ? k_fft64_lines<1, true, 1024, 8192> : k_fft64_lines<1, false, 1024, 8192>)
                     : (out_c64 ? k_fft64_lines<-1, true, 1024, 8192> : k_fft64_lines<-1, false, 1024, 8192>);
    else
        kern = S > 0 ? (out_c64 ? k_fft64_lines<1, true, 512, 4096> : k_fft64_lines<1, false, 512, 4096>)
                     : (out_c64 ? k_fft64_lines<-1, true, 512, 4096> : k_fft64_lines<-1, false, 512, 4096>);
    if (lds > 65536)
        MN_HIP_CHECK(hipFuncSetAttribute((const void *)kern,
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    kern<<<(unsigned)ntiles, longl ? 1024 : 512, lds, s>>>(static_cast<const double2 *>(in), out,
                                                          dec, tw, nlines, (int)B, (int)Bo,
                                                          ntiles, p);
    MN_LAUNCH_CHECK("fft64_lines");
    return MN_OK;
}

int mn_transpose_c128(int64_t Bt, int64_t R, int64_t C, const void *in, void *out,
                      mn_stream_t stream) {
    clear_error();
    MN_REQUIRE(in && out && in != out, "transpose: NULL or aliased buffers");
    MN_REQUIRE(Bt >= 1 && Bt <= 65535 && R >= 1 && C >= 1 && R < (int64_t(1) << 31) &&
                   C < (int64_t(1) << 31) && (R + 31) / 32 <= 65535,
               "transpose: shape out of range");
    const dim3 grid((unsigned)((C + 31) / 32), (unsigned)((R + 31) / 32), (unsigned)Bt);
    k_transpose_c128<<<grid, 256, 0, as_stream(stream)>>>(static_cast<const double2 *>(in),
                                                         static_cast<double2 *>(out), (int)R,
                                                         (int)C);
    MN_LAUNCH_CHECK("transpose");
    return MN_OK;
}

}  // extern "C"
