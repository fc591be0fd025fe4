// 2D owner-computes spread on the matrix cores ("y-window MFMA sweep"): the
// 2D counterpart of the z-sweep (mn_zsweep.hip). No atomics; every
// fine-grid cell is written exactly once with a plain store.
//
// Layout. The grid (n0 x n1, n1 contiguous) is cut into blocks of 16
// consecutive x-columns. One wavefront owns a block over a y-segment (a
// multiple of 8 cells) for VB strength vectors and sweeps it upwards in
// y-chunks of 8 cells. Per vector the block's window is one
// v_mfma_f32_16x16x32_f16 accumulator tile for the real and one for the
// imaginary part: rows are the 16 x-columns, columns 16 consecutive y-slots
// (the chunk being processed, slots 0..7, and the 8 cells above it, which
// the footprints of the chunk's points reach).
//
// Matrix form. For a K-step of 32 points p,
//   D[x][s] += sum_p wx_p[x] * (c_p wy_p[s])
// with A = the x-weights (fp16 hi and lo, formed once per point in the
// prologue) and B = the strength times the y-weight, formed per vector in
// the K-step and split into fp16 hi and lo there: hi*hi' + hi*lo' + lo*hi'
// carries the f32 product to about 2^-22 (the z-sweep's scheme, with the
// x-y product replaced by the strength-y product).
//
// Point order. Points are sorted by the key of the (block, chunk) of their
// first tap and a reach bit (ym_word); a block takes its own points (both
// reach values) and the reaching points of its -x neighbour: two contiguous
// key ranges per chunk, found through ystart (first sorted index with a key
// at or above k). The word carries the first tap's x cell in its block and
// y cell in its chunk.
//
// Batches of up to 64 points (a lane per point): the rest of the current
// chunk (part A) and, when that ends first, the head of the next chunk from
// the next multiple of 8 lanes (part B), as in the z-sweep. The prologue
// writes the point's W x-weights into its column of the A tables ([x][point],
// taps off the block into junk rows that are never read), its W y-weights
// into the y table ([slot][point]) and its scaled strengths into the
// strength table ([vector][point]); the tables' zero group (positions 64..71)
// is what K-step lanes past a batch part read.
//
// Strengths. c holds B rows of P (vector-major) or P rows of B
// (point-major): with several vectors the point-major layout puts a point's
// strengths in one run, one sector per point visit instead of one per
// vector (the gathers bound the vector-major spread: at 8 vectors a visit
// touched 8 random sectors).
//
// Scale. A carries 2^14 and B a per-vector power of two 2^s with
// |c 2^s| < 2^14 (the z-sweep's rule), so any finite fp32 strength keeps
// the fp16 operands normal; results are unscaled by ldexp at the store.
//
// ref: nd.py:492-579 (the reference's output-driven spread this replaces),
// nd.py:683-742 (its batched spread), nd.py:298-372 (bin sort).
#include "mn_common.h"
#include "mn_zsweep.h"

namespace mn {
namespace {

constexpr int XB = kYmBlock;  // x-columns per block
constexpr int YC = kYmChunk;  // y-cells per chunk
constexpr int NR = 2;         // key ranges per chunk: own block, -x neighbour (reaching)
constexpr int kZeroGroup = 8;  // positions 64..71: zero A columns
// A tables: rows x + AJ for x in [-AJ, XB + AJ) (taps off the block land in
// the junk rows), 72 halves per row (64 points and the zero group; rows 36
// dwords apart put the 16 rows of a quarter-wave's 16-byte reads on
// distinct banks)
constexpr int AJ = 7;
constexpr int AROWS = XB + 2 * AJ;
constexpr int ATS = 72;
// y table: 16 slot rows of 76 floats (64 points, the zero group, 4 of
// padding: rows 12 banks apart keep a quarter-wave's 16-byte reads apart)
constexpr int YTS = 76;
constexpr int CTS = 72;  // float2 per strength row
constexpr float kAScale = 16384.0f;  // 2^14 on the x-weights

typedef float mf4 __attribute__((ext_vector_type(4)));
typedef float mf2 __attribute__((ext_vector_type(2)));
typedef _Float16 mh8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float row_shl8_zero(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x108, 0xf, 0xf, true));
}

// hi/lo fp16 halves of the products x[t] y[t] (t = 0..7): hi is the f32
// product rounded toward zero, lo = fp16(fma(x, y, -hi)) (mixed-precision
// fmas reading hi as fp16)
__device__ __forceinline__ void split_prod8(const float (&x)[8], const float (&y)[8], mh8 &hi,
                                            mh8 &lo) {
    typedef _Float16 mh2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int t = 0; t < 8; t += 2) {
        const auto h = __builtin_amdgcn_cvt_pkrtz(x[t] * y[t], x[t + 1] * y[t + 1]);
        hi[t] = h[0];
        hi[t + 1] = h[1];
        uint32_t hb, lb;
        __builtin_memcpy(&hb, &h, 4);
        asm("v_fma_mixlo_f16 %0, %1, %2, -%3 op_sel_hi:[0,0,1]\n\t"
            "v_fma_mixhi_f16 %0, %4, %5, -%3 op_sel:[0,0,1] op_sel_hi:[0,0,1]"
            : "=&v"(lb)
            : "v"(x[t]), "v"(y[t]), "v"(hb), "v"(x[t + 1]), "v"(y[t + 1]));
        mh2 l;
        __builtin_memcpy(&l, &lb, 4);
        lo[t] = l[0];
        lo[t + 1] = l[1];
    }
}

// The two key ranges of a chunk: range 0 = the block's own points, range 1
// = the -x neighbour's reaching points.
struct YmRanges {
    int bx, dbx, nyc, clast;
    const int32_t *ystart;
    // (st, en) of range `lane` (lanes 0, 1) of chunk c (c = -1 is the last
    // chunk, periodically); an empty range (both ystart[0]) for other lanes
    // and for chunks past clast. The loaded values are returned as they are.
    __device__ __forceinline__ int2 fetch(int c, int lane) const {
        const int r = lane & 1;
        const bool ok = lane < NR && c <= clast;
        const int cc = c < 0 ? c + nyc : c;
        const int64_t kb = ok ? ((int64_t)(bx + r * dbx) * nyc + cc) * 2 : 0;
        return make_int2(ystart[kb + (ok ? r : 0)], ystart[kb + (ok ? 2 : 0)]);
    }
};

// The wave's position in the chunks of its segment (uniform): the current
// chunk c, its next batch element and element count, the range boundary p1
// and offsets dj0, dj1 (sorted index = element + dj of its range), and the
// prefetched bounds of chunk pc.
struct YmCursor {
    int c, clast, bat, tot;
    int p1, dj0, dj1;
    int pc, nst, nen;
};

__device__ __forceinline__ void ym_fetch(YmCursor &k, const YmRanges &rg, int c, int lane) {
    const int2 b = rg.fetch(c, lane);
    k.pc = c;
    k.nst = b.x;
    k.nen = b.y;
}

// Make chunk c current and start fetching the bounds of chunk c + 1.
__device__ __forceinline__ void ym_load(YmCursor &k, const YmRanges &rg, int c, int lane) {
    if (k.pc != c) ym_fetch(k, rg, c, lane);
    const int st0 = __builtin_amdgcn_readlane(k.nst, 0), n0 = __builtin_amdgcn_readlane(k.nen, 0) - st0;
    const int st1 = __builtin_amdgcn_readlane(k.nst, 1), n1 = __builtin_amdgcn_readlane(k.nen, 1) - st1;
    k.c = c;
    k.bat = 0;
    k.p1 = n0;
    k.tot = n0 + n1;
    k.dj0 = st0;
    k.dj1 = st1 - n0;
    ym_fetch(k, rg, c + 1, lane);
}

// One lane's point of a batch, its loads issued (the strengths, which need
// src, are loaded one batch later).
struct YmPoint {
    int cA, nA, cB, oB, nB;  // uniform; nA = 0: done
    bool valid, inB;
    int r;                   // the point's range (source block)
    uint32_t wd, src;        // sorted word; index of its strength in c
    float fx, fy;
};

__device__ __forceinline__ YmPoint ym_next(YmCursor &k, const YmRanges &rg, int lane,
                                           const uint32_t *__restrict__ perm,
                                           const uint32_t *__restrict__ word,
                                           const float *__restrict__ frx,
                                           const float *__restrict__ fry) {
    // past exhausted (or empty) chunks: usually one step, straight-line code
    if (k.bat >= k.tot && k.c <= k.clast) {
        ym_load(k, rg, k.c + 1, lane);
        while (k.bat >= k.tot && k.c <= k.clast) ym_load(k, rg, k.c + 1, lane);
    }
    YmPoint q;
    q.cA = k.c;
    q.nA = k.c <= k.clast ? min(64, k.tot - k.bat) : 0;
    q.cB = k.c + 1;
    q.oB = (q.nA + 7) & ~7;
    q.nB = 0;
    // part A: elements bat + lane of the current chunk
    const int eA = k.bat + lane;
    int r = eA >= k.p1 ? 1 : 0;
    int dj = r == 0 ? k.dj0 : k.dj1;
    int e = eA;
    k.bat += q.nA;
    if (q.nA > 0 && q.oB < 64 && k.c + 1 <= k.clast) {
        // part B: the head of the next chunk, whose bounds were prefetched
        ym_load(k, rg, k.c + 1, lane);
        q.nB = min(64 - q.oB, k.tot);
        k.bat = q.nB;
        if (lane >= q.oB) {
            e = lane - q.oB;
            r = e >= k.p1 ? 1 : 0;
            dj = r == 0 ? k.dj0 : k.dj1;
        }
    }
    q.inB = lane >= q.oB;
    q.valid = lane < q.nA || (q.inB && lane < q.oB + q.nB);
    const uint32_t j = q.valid ? (uint32_t)(e + dj) : 0u;
    q.r = r;
    q.wd = word[j];
    q.fx = frx[j];
    q.fy = fry[j];
    const uint32_t pj = (perm ? perm : word)[j];
    q.src = perm ? pj : j;
    return q;
}

template <int W, int VB>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2))) void
k_spread_ymfma(int n1, int nbx, int nyc, int yseg, int nseg, float bl2e,
               const int32_t *__restrict__ ystart, const uint32_t *__restrict__ perm,
               const uint32_t *__restrict__ word, const float *__restrict__ frx,
               const float *__restrict__ fry, const float2 *__restrict__ c, int64_t cvs,
               int64_t cps, int64_t B, float2 *__restrict__ grid, int64_t gstride) {
    static_assert(W >= 2 && W <= 8 && YC + W - 1 <= 16, "footprint exceeds the 16 slots");
    static_assert(W - 1 <= AJ, "junk rows too few");
    __shared__ __align__(16) _Float16 atab[2][AROWS * ATS];  // x-weights hi, lo
    __shared__ __align__(16) float ytab[16 * YTS];            // y-weights by slot
    __shared__ __align__(16) float2 ctab[VB][CTS];            // scaled strengths

    // blocks fastest: a block and its -x neighbour, which read the same
    // reaching points, run on one XCD at about the same y
    const int wid = (int)xcd_remap(blockIdx.x, (int64_t)nbx * nseg);
    const int bx = wid % nbx, seg = wid / nbx;
    const int bxm = bx == 0 ? nbx - 1 : bx - 1;
    const int64_t v0 = (int64_t)blockIdx.y * VB;
    const int nv = (int)min((int64_t)VB, B - v0);  // vectors of this wave (>= 1)
    c += v0 * cvs;
    grid += v0 * gstride;
    const int y0 = seg * yseg, yend = min(y0 + yseg, n1);
    const int lane = threadIdx.x, li = lane & 15, lk = lane >> 4;
    int sexp[VB];  // INT32_MIN: unset until the first batch
    mf4 are[VB], aim[VB];
#pragma unroll
    for (int v = 0; v < VB; ++v) {
        sexp[v] = INT32_MIN;
        are[v] = mf4{0.f, 0.f, 0.f, 0.f};
        aim[v] = mf4{0.f, 0.f, 0.f, 0.f};
    }
    int yb = y0 - YC;  // y of slot 0
    // cells (16 bx + 4 lk + i, y) for i < 4: a uniform base per i plus the
    // lane's byte offset
    const int64_t gcol = (int64_t)(XB * bx + 4 * lk) * n1;

    // Slots 0..7 are complete: store the owned ones, shift the window by 8.
    auto advance = [&]() __attribute__((always_inline)) {
        const int y = yb + li;
        if (li < YC && y >= y0 && y < yend) {
#pragma unroll
            for (int v = 0; v < VB; ++v) {
                if (v >= nv) break;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const mf2 val = {__builtin_amdgcn_ldexpf(are[v][i], -14 - sexp[v]),
                                     __builtin_amdgcn_ldexpf(aim[v][i], -14 - sexp[v])};
                    __builtin_nontemporal_store(
                        val, reinterpret_cast<mf2 *>(grid + v * gstride + gcol + (int64_t)i * n1 + y));
                }
            }
        }
#pragma unroll
        for (int v = 0; v < VB; ++v)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                are[v][i] = row_shl8_zero(are[v][i]);
                aim[v][i] = row_shl8_zero(aim[v][i]);
            }
        yb += YC;
    };

    // the window moves up to chunk c: usually one step, straight-line code
    auto window_to = [&](int c) __attribute__((always_inline)) {
        const int yt = YC * c;
        if (yb < yt) {
            advance();
            if (yb < yt) {
                advance();
                while (yb < yt) advance();
            }
        }
    };

    // K-steps of 32 points over the 8-point groups [g0, g1) of the tables;
    // lanes past g1 read the zero group (zero A columns)
    auto ksteps = [&](int g0, int g1) __attribute__((always_inline)) {
        for (int gs = g0; gs < g1; gs += 4) {
            const int pos = 8 * (gs + lk < g1 ? gs + lk : kZeroGroup);
            const mh8 ah = *reinterpret_cast<const mh8 *>(&atab[0][(AJ + li) * ATS + pos]);
            const mh8 al = *reinterpret_cast<const mh8 *>(&atab[1][(AJ + li) * ATS + pos]);
            float wy[8];
            {
                const float4 y0v = *reinterpret_cast<const float4 *>(&ytab[li * YTS + pos]);
                const float4 y1v = *reinterpret_cast<const float4 *>(&ytab[li * YTS + pos + 4]);
                wy[0] = y0v.x, wy[1] = y0v.y, wy[2] = y0v.z, wy[3] = y0v.w;
                wy[4] = y1v.x, wy[5] = y1v.y, wy[6] = y1v.z, wy[7] = y1v.w;
            }
#pragma unroll
            for (int v = 0; v < VB; ++v) {
                float cr[8], ci[8];
#pragma unroll
                for (int t = 0; t < 8; t += 2) {
                    const float4 cc = *reinterpret_cast<const float4 *>(&ctab[v][pos + t]);
                    cr[t] = cc.x, ci[t] = cc.y, cr[t + 1] = cc.z, ci[t + 1] = cc.w;
                }
                mh8 brh, brl, bih, bil;
                split_prod8(cr, wy, brh, brl);
                split_prod8(ci, wy, bih, bil);
                are[v] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, brh, are[v], 0, 0, 0);
                aim[v] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bih, aim[v], 0, 0, 0);
                are[v] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, brl, are[v], 0, 0, 0);
                aim[v] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bil, aim[v], 0, 0, 0);
                are[v] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, brh, are[v], 0, 0, 0);
                aim[v] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bih, aim[v], 0, 0, 0);
            }
        }
    };

    auto process = [&](const YmPoint &p, const float2 (&cp)[VB]) __attribute__((always_inline)) {
        const bool valid = p.valid;
#pragma unroll
        for (int v = 0; v < VB; ++v) {
            // the scale is lowered when a strength reaches 2^(141 - sexp - 127);
            // then the batch's largest strength is below 2^(e - 126)
            const float2 cv = valid ? cp[v] : make_float2(0.f, 0.f);
            const float mx = fmaxf(fabsf(cv.x), fabsf(cv.y));
            const int eb = (__float_as_int(mx) >> 23) & 0xff;
            if (sexp[v] == INT32_MIN || __ballot(eb > 140 - sexp[v])) {
                const int want = min(140 - wave_max9(eb), 139);
                if (sexp[v] != INT32_MIN) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        are[v][i] = __builtin_amdgcn_ldexpf(are[v][i], want - sexp[v]);
                        aim[v][i] = __builtin_amdgcn_ldexpf(aim[v][i], want - sexp[v]);
                    }
                }
                sexp[v] = want;  // below the old scale whenever one was set
            }
        }
        window_to(p.cA);
        // the wave's LDS operations complete in issue order; compiler-only
        // fences keep the tables' program order around the K-steps' reads
        asm volatile("" ::: "memory");
        {
            // zero the 16 x rows (both halves) and the 16 slot rows at the
            // batch positions 0..63; the junk rows are never read
            float4 *a4 = reinterpret_cast<float4 *>(&atab[0][0]);
            constexpr int arow4 = ATS / 8;  // float4 per A row
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int i = lane + 64 * k;  // 256 = 2 tables x 16 rows x 8 float4
                const int t = i >> 7, row = (i >> 3) & 15, col = i & 7;
                a4[(t * AROWS + AJ + row) * arow4 + col] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int i = lane + 64 * k;  // 256 = 16 rows x 16 float4
                reinterpret_cast<float4 *>(&ytab[(i >> 4) * YTS])[i & 15] =
                    make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        asm volatile("" ::: "memory");
#pragma unroll
        for (int v = 0; v < VB; ++v)
            ctab[v][lane] = valid ? make_float2(__builtin_amdgcn_ldexpf(cp[v].x, sexp[v]),
                                                __builtin_amdgcn_ldexpf(cp[v].y, sexp[v]))
                                  : make_float2(0.f, 0.f);
        if (valid) {
            // first tap relative to this block (minus 16 for points of the
            // -x neighbour) and its slot in its chunk's window
            const int ox = (int)((p.wd >> kYmKeyBits) & 15u) - ((p.r & 1) ? XB : 0);
            const int sy = (int)(p.wd >> 29);
            _Float16 *ah = &atab[0][(AJ + ox) * ATS + lane];
            _Float16 *al = &atab[1][(AJ + ox) * ATS + lane];
            float *wyc = &ytab[sy * YTS + lane];
            constexpr float ih = 2.0f / W;
#pragma unroll
            for (int a = 0; a < W; ++a) {
                const float ca = (float)a * ih;
                const float wx = zs_es(__builtin_fmaf(-p.fx, ih, ca), bl2e) * kAScale;
                const auto h = __builtin_amdgcn_cvt_pkrtz(wx, 0.f);
                ah[a * ATS] = h[0];
                al[a * ATS] = (_Float16)(wx - (float)h[0]);
                wyc[a * YTS] = zs_es(__builtin_fmaf(-p.fy, ih, ca), bl2e);
            }
        }
        asm volatile("" ::: "memory");
        // part A in its chunk's window, then part B in the next chunk's
        ksteps(0, (p.nA + 7) >> 3);
        if (p.nB > 0) {
            window_to(p.cB);
            ksteps(p.oB >> 3, (p.oB + p.nB + 7) >> 3);
        }
        asm volatile("" ::: "memory");
    };

    auto strengths = [&](const YmPoint &p, float2 (&cv)[VB]) __attribute__((always_inline)) {
#pragma unroll
        for (int v = 0; v < VB; ++v) cv[v] = c[(int64_t)min(v, nv - 1) * cvs + (int64_t)p.src * cps];
    };

    // the tables' zero group (never written by a batch) and the strength
    // table's, which K-step lanes past a part read
    for (int i = lane; i < 2 * AROWS * ATS; i += 64) (&atab[0][0])[i] = (_Float16)0.f;
    for (int i = lane; i < 16 * YTS; i += 64) ytab[i] = 0.f;
#pragma unroll
    for (int v = 0; v < VB; ++v)
        for (int i = lane; i < CTS; i += 64) ctab[v][i] = make_float2(0.f, 0.f);
    asm volatile("" ::: "memory");

    const int clast = (yend - 1) / YC;  // the last chunk of the segment
    const YmRanges rg{bx, bxm - bx, nyc, clast, ystart};
    YmCursor cur;
    cur.pc = INT32_MIN;
    cur.clast = clast;
    ym_load(cur, rg, y0 / YC - 1, lane);
    YmPoint pa = ym_next(cur, rg, lane, perm, word, frx, fry);
    float2 ca[VB], cb[VB], cc[VB];
    strengths(pa, ca);  // idle lanes read c[perm[0]]: their columns stay zero
    YmPoint pb = ym_next(cur, rg, lane, perm, word, frx, fry);
    YmPoint pc;
    for (;;) {
        if (pa.nA == 0) break;
        pc = ym_next(cur, rg, lane, perm, word, frx, fry);
        strengths(pb, cb);
        process(pa, ca);
        if (pb.nA == 0) break;
        pa = ym_next(cur, rg, lane, perm, word, frx, fry);
        strengths(pc, cc);
        process(pb, cb);
        if (pc.nA == 0) break;
        pb = ym_next(cur, rg, lane, perm, word, frx, fry);
        strengths(pa, ca);
        process(pc, cc);
    }
#pragma unroll
    for (int v = 0; v < VB; ++v)
        if (sexp[v] == INT32_MIN) sexp[v] = 0;  // no points at all: the window holds zeros
    while (yb < yend) advance();
}

struct YmArgs {
    int n1, nbx, nyc, yseg, nseg;
    float bl2e;
    int64_t P, B, gsz, cvs, cps;
    const int32_t *ystart;
    const uint32_t *perm, *word;
    const float *fx, *fy;
    const float2 *c;
    float2 *grid;
    hipStream_t s;
};

// Vectors per wave: the largest of 8, 4, 2, 1 not above B.
inline int ym_vb(int64_t B) { return B >= 8 ? 8 : (B >= 4 ? 4 : (B >= 2 ? 2 : 1)); }

template <int W, int VB>
int ym_launch_vb(const YmArgs &a) {
    const dim3 blocks((unsigned)(a.nbx * a.nseg), (unsigned)((a.B + VB - 1) / VB));
    k_spread_ymfma<W, VB><<<blocks, 64, 0, a.s>>>(a.n1, a.nbx, a.nyc, a.yseg, a.nseg, a.bl2e,
                                                  a.ystart, a.perm, a.word, a.fx, a.fy, a.c, a.cvs,
                                                  a.cps, a.B, a.grid, a.gsz);
    MN_LAUNCH_CHECK("spread_ymfma");
    return MN_OK;
}

template <int W>
int ym_launch(const YmArgs &a) {
    switch (ym_vb(a.B)) {
        case 8: return ym_launch_vb<W, 8>(a);
        case 4: return ym_launch_vb<W, 4>(a);
        case 2: return ym_launch_vb<W, 2>(a);
        default: return ym_launch_vb<W, 1>(a);
    }
}

}  // namespace

int ymfma_check(const mn_bins *g) {
    MN_REQUIRE(g != nullptr && g->dim == 2, "ymfma: 2D geometry required");
    MN_REQUIRE(g->w >= 2 && g->w <= 8, "ymfma: kernel width must be in [2, 8]");
    MN_REQUIRE(g->n[0] % XB == 0 && g->n[0] >= 2 * XB, "ymfma: n0 must be a multiple of 16, >= 32");
    MN_REQUIRE(g->n[1] % YC == 0 && g->n[1] >= 2 * YC && g->n[1] < (int64_t(1) << 24),
               "ymfma: n1 must be a multiple of 8 in [16, 2^24)");
    MN_REQUIRE(ymfma_nkeys(g) <= (int64_t(1) << kYmKeyBits), "ymfma: key space above 2^25");
    return MN_OK;
}

int64_t ymfma_nkeys(const mn_bins *g) { return (g->n[0] / XB) * (g->n[1] / YC) * 2; }

namespace {

// Vector-major (B, P) complex64 strengths to point-major (P, B).
// For B in {2, 4, 8} a 256-thread workgroup stages PM_TP points of all B rows
// in LDS: every global load instruction reads 64 consecutive values of one
// row and every store instruction writes 64 consecutive output values, so
// both sides stream; the LDS tile is point-major with a one-value pad per
// point (stride B + 1 values: B = 8 puts a wave's scattered tile writes on
// 2-way banks). Other B take a lane per output element.
// (Measured at B = 8, P = 1e7: a lane per output element 0.23 ms, its
// loads gathering 8 row segments per instruction; a thread per point
// writing its 64-byte run with four 16-byte stores 0.29 ms; torch's
// transpose 0.25 ms.)
constexpr int PM_THREADS = 256;
constexpr int PM_ITEMS = 8;   // values per thread
template <int BV>
__global__ __launch_bounds__(PM_THREADS) void k_pointmajor_tile(int64_t P,
                                                                const float2 *__restrict__ in,
                                                                float2 *__restrict__ out) {
    constexpr int TP = PM_THREADS * PM_ITEMS / BV;  // points per tile
    __shared__ float2 tile[TP * (BV + 1)];
    const int64_t p0 = (int64_t)blockIdx.x * TP;
    const int t = threadIdx.x;
    float2 v[PM_ITEMS];
    // value i of thread t: row (i * 256 + t) / TP, point (i * 256 + t) % TP
#pragma unroll
    for (int i = 0; i < PM_ITEMS; ++i) {
        const int q = i * PM_THREADS + t, b = q / TP, pl = q % TP;
        const int64_t p = p0 + pl;
        v[i] = p < P ? in[(int64_t)b * P + p] : make_float2(0.f, 0.f);
    }
#pragma unroll
    for (int i = 0; i < PM_ITEMS; ++i) {
        const int q = i * PM_THREADS + t, b = q / TP, pl = q % TP;
        tile[pl * (BV + 1) + b] = v[i];
    }
    __syncthreads();
    // output element e = p0 B + q: point q / B, row q % B
    const int64_t nout = (P - p0 < TP ? P - p0 : TP) * BV;
#pragma unroll
    for (int i = 0; i < PM_ITEMS; ++i) {
        const int q = i * PM_THREADS + t;
        if (q < nout) out[p0 * BV + q] = tile[(q / BV) * (BV + 1) + q % BV];
    }
}
template <int BV>
__global__ __launch_bounds__(PM_THREADS) void k_pointmajor_c64(int64_t B, int64_t P,
                                                               const float2 *__restrict__ in,
                                                               float2 *__restrict__ out) {
    const int64_t nb = BV > 0 ? BV : B;
    const int64_t n = nb * P;
    const int64_t e0 = (int64_t)blockIdx.x * (PM_THREADS * PM_ITEMS) + threadIdx.x;
    float2 v[PM_ITEMS];
#pragma unroll
    for (int i = 0; i < PM_ITEMS; ++i) {
        const int64_t e = e0 + (int64_t)i * PM_THREADS;
        const int64_t p = e / nb, b = e - p * nb;
        v[i] = e < n ? in[b * P + p] : make_float2(0.f, 0.f);
    }
#pragma unroll
    for (int i = 0; i < PM_ITEMS; ++i) {
        const int64_t e = e0 + (int64_t)i * PM_THREADS;
        if (e < n) out[e] = v[i];
    }
}

}  // namespace

}  // namespace mn

using namespace mn;

extern "C" {

int64_t mn_ymfma_nkeys(const mn_bins *g) {
    clear_error();
    if (ymfma_check(g)) return -1;
    return ymfma_nkeys(g);
}

int mn_ymfma_starts(const mn_bins *g, int64_t P, const uint32_t *sorted_word, int32_t *ystart,
                    mn_stream_t stream) {
    clear_error();
    int rc = ymfma_check(g);
    if (rc) return rc;
    MN_REQUIRE(P >= 1 && P < (int64_t(1) << 31), "ymfma starts: P must be in [1, 2^31)");
    MN_REQUIRE(sorted_word && ystart, "ymfma starts: NULL pointer");
    return key_starts(sorted_word, P, ymfma_nkeys(g), kYmKeyMask, ystart, as_stream(stream));
}

int mn_spread_ymfma(const mn_bins *g, float beta, int64_t P, int64_t B, int yseg,
                    const int32_t *ystart, const uint32_t *perm, const uint32_t *sorted_word,
                    const float *const frs[2], const void *c, int point_major, void *grid,
                    mn_stream_t stream) {
    clear_error();
    int rc = ymfma_check(g);
    if (rc) return rc;
    MN_REQUIRE(P >= 1 && P < (int64_t(1) << 31), "ymfma spread: P must be in [1, 2^31)");
    MN_REQUIRE(B >= 1 && B <= 65535, "ymfma spread: B must be in [1, 65535]");
    MN_REQUIRE(yseg >= YC && yseg % YC == 0, "ymfma spread: yseg must be a positive multiple of 8");
    MN_REQUIRE(ystart && sorted_word && frs && frs[0] && frs[1] && c && grid,
               "ymfma spread: NULL pointer");
    YmArgs a{};
    a.n1 = (int)g->n[1];
    a.nbx = (int)(g->n[0] / XB);
    a.nyc = (int)(g->n[1] / YC);
    a.yseg = yseg;
    a.nseg = (int)((g->n[1] + yseg - 1) / yseg);
    MN_REQUIRE((int64_t)a.nbx * a.nseg < (int64_t(1) << 31), "ymfma spread: too many blocks");
    a.bl2e = (float)(beta * 1.4426950408889634);
    a.P = P;
    a.B = B;
    a.gsz = g->n[0] * g->n[1];
    // strength of point i in vector v: c[v * cvs + i * cps]
    a.cvs = point_major ? 1 : P;
    a.cps = point_major ? B : 1;
    a.ystart = ystart;
    a.perm = perm;
    a.word = sorted_word;
    a.fx = frs[0];
    a.fy = frs[1];
    a.c = static_cast<const float2 *>(c);
    a.grid = static_cast<float2 *>(grid);
    a.s = as_stream(stream);
    switch (g->w) {
        case 2: return ym_launch<2>(a);
        case 3: return ym_launch<3>(a);
        case 4: return ym_launch<4>(a);
        case 5: return ym_launch<5>(a);
        case 6: return ym_launch<6>(a);
        case 7: return ym_launch<7>(a);
        case 8: return ym_launch<8>(a);
    }
    set_error("ymfma spread: kernel width must be in [2, 8]");
    return MN_EINVAL;
}

int mn_pointmajor_c64(int64_t B, int64_t P, const void *in, void *out, mn_stream_t stream) {
    clear_error();
    MN_REQUIRE(B >= 1 && B < 65536 && P >= 1 && P < (int64_t(1) << 40) &&
                   B * P / PM_ITEMS / PM_THREADS < (int64_t(1) << 31),
               "pointmajor: B must be in [1, 65535], P in [1, 2^40) and B P below 2^42");
    MN_REQUIRE(in && out && in != out, "pointmajor: NULL or aliased pointer");
    const float2 *ci = static_cast<const float2 *>(in);
    float2 *co = static_cast<float2 *>(out);
    const unsigned nblk =
        (unsigned)((B * P + PM_THREADS * PM_ITEMS - 1) / (PM_THREADS * PM_ITEMS));
    hipStream_t s = as_stream(stream);
    auto tiles = [&](int bv) { return (unsigned)((P * bv + PM_THREADS * PM_ITEMS - 1) /
                                                 (PM_THREADS * PM_ITEMS)); };
    switch (B) {
        case 2: k_pointmajor_tile<2><<<tiles(2), PM_THREADS, 0, s>>>(P, ci, co); break;
        case 4: k_pointmajor_tile<4><<<tiles(4), PM_THREADS, 0, s>>>(P, ci, co); break;
        case 8: k_pointmajor_tile<8><<<tiles(8), PM_THREADS, 0, s>>>(P, ci, co); break;
        default: k_pointmajor_c64<0><<<nblk, PM_THREADS, 0, s>>>(B, P, ci, co); break;
    }
    MN_LAUNCH_CHECK("pointmajor_c64");
    return MN_OK;
}

}  // extern "C"
