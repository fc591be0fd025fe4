// Z-gather interpolation (3D type-2 core): every point is visited once, by
// the wavefront that owns the 8x8 column block and z-chunk of its first tap,
// with the grid window on the matrix cores and no per-tap gathers.
//
// Points. Words and fractions sorted by the key of the first tap's (block,
// z-chunk) as for the z-sweep spread (mn_zsweep.hip), but with the points of
// a (block, chunk) ordered by the x cell of their first tap (zg_word): the
// points one wave owns over its z-segment are one contiguous run of the
// sorted arrays, chunk by chunk, bounded through zstart, and the 16 points of
// a tile cover a narrow run of x columns, so the tile skips the MFMAs and
// wx sums of the columns none of them reaches. Their footprints lie
// in the window of NX = 8 + w - 1 columns per axis (x = 8 bx + X,
// y = 8 by + Y, periodic). Along z the points of chunk c reach
// [8c, 8c + 8 + w - 1), inside the 16 cells [8c, 8c + 16) that the wave
// holds as a ring of 16 z-slots (slot = z mod 16): moving up one chunk
// replaces the slots of z-run 8(c - 1) by z-run 8(c + 1).
//
// Matrix form. For a tile of 16 points p and each window column X,
//   C_X[p][n] = sum_Y wy_p[Y] G[X][Y][z(n)]        (n = ring slot)
// is one 16x16 product with K = Y (rows past NX zero), and
//   out[p] = sum_n wz_p[z(n)] sum_X wx_p[X] C_X[p][n].
// The window is the B operand of v_mfma_f32_16x16x32_f16, kept in registers
// for the whole sweep: for each X, lane (n, g) (n = l % 16, g = l / 16)
// holds B[k = 8g + i][n] for i < 8, the fp16 hi half of G[X][k][z(n)] for
// k < 16 and the lo half of G[X][k - 16][z(n)] for k >= 16, both scaled by
// 2^s (one power of two per ring half, so that the half's largest value is
// below 2^15). With A1 = [wy_hi | wy_hi] and A2 = [wy_lo | 0] (wy scaled by
// 2^14 and split likewise), A1 B + A2 B = hi*hi + hi*lo + lo*hi with every
// product exact in f32: four MFMAs per X for the real and imaginary parts.
// The wx sum runs on the accumulator layout (lane (n, g) holds rows 4g + i
// of column n), the wz weights and the scales multiply it, and a
// reduce-scatter over each 8 lanes of a row (then a sum of the two halves)
// leaves each of the tile's 8 results (4 points x re, im) in two lanes; the
// lane holding a point's real part takes the imaginary part from its DPP
// partner and stores the pair as one 8-byte value.
//
// Batches. Up to 64 points (a lane per point): the prologue evaluates the
// point's 3w ES weights once and writes the tables the tiles read -- its A
// row (wy hi and lo at Y = oy + a), its wx column ([X][point]) and its wz
// column by ring slot ([slot][point]), zeros elsewhere. A batch holds the
// rest of one chunk (part A) and, when that ends early, the head of the next
// non-empty chunk (part B, from the next multiple of 16 lanes), so tiles run
// nearly full; the window moves between the two parts.
//
// Window loads. The 8 new z-cells of the NX x NX columns are read as 64-byte
// runs (lane: z-cell l % 8 of Y pair l / 8), scaled, split into hi and lo,
// staged in LDS in the B layout and read back (16 bytes per lane and X) by
// the lanes of the ring half they replace; the real and imaginary parts take
// turns in one staging buffer. LDS operations of a wave complete in issue
// order, so the one-wave workgroup needs no barrier between a table's reads
// and its next writes.
// ref: nd.py:974-1073 (the reference's output-driven gather this replaces),
// nd.py:298-372 (its bin sort).
#include <type_traits>

#include "mn_common.h"
#include "mn_zsweep.h"

namespace mn {
namespace {

constexpr int ZB = kZsBlock;
constexpr int ZC = kZsChunk;
// halves per A row: wy hi at Y (0..15), lo at 16 + Y, then 8 of padding:
// 80-byte rows put the 8 lanes of a 16-byte read phase on disjoint banks
constexpr int AROW = 40;
// floats per wx / wz table row: 64 points + 4 (the slot rows that one wz
// read phase touches start 4 banks apart)
constexpr int TROW = 68;

typedef float gf4 __attribute__((ext_vector_type(4)));
typedef _Float16 gh8 __attribute__((ext_vector_type(8)));

// v moved across lanes by a DPP pattern (every source lane is in range)
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
constexpr int kDppRowRor8 = 0x128;        // lane n <- n ^ 8 within a row of 16
constexpr int kDppRowHalfMirror = 0x141;  // lane n <- 7 - n within 8
constexpr int kDppQuadMirror = 0x1b;      // quad_perm [3, 2, 1, 0]
constexpr int kDppQuadSwap = 0xb1;        // quad_perm [1, 0, 3, 2]

// lo halves of the pair (a, b) given their hi halves (cvt_pkrtz): f16(a -
// hi.x), f16(b - hi.y), each one fused multiply-add with the f16 operand
// converted in the instruction
__device__ __forceinline__ uint32_t split_lo(float a, float b, uint32_t hi) {
    uint32_t lo;
    asm("v_fma_mixlo_f16 %0, %1, 1.0, -%2 op_sel_hi:[0,0,1]\n\t"
        "v_fma_mixhi_f16 %0, %3, 1.0, -%2 op_sel:[0,0,1] op_sel_hi:[0,0,1]"
        : "=&v"(lo)
        : "v"(a), "v"(hi), "v"(b));
    return lo;
}

// 32-bit LDS address of a __shared__ object
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// v = 16 bytes of LDS at address a + OFF, written in place (lanes the exec
// mask leaves out keep v); the caller waits (lgkmcnt) before using v
template <typename T>
__device__ __forceinline__ void ds_read_b128_into(T &v, uint32_t a, const int off) {
    static_assert(sizeof(T) == 16, "16-byte operand");
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "+v"(v) : "v"(a), "i"(off) : "memory");
}

// The uniform description of a batch and one lane's loads for it.
struct ZgBatch {
    int cA, jA, nA, oB, jB, nB, cB;  // nA = 0: no batch
};
struct ZgPoint {
    uint32_t wd, pj;
    float fx, fy, fz;
};

template <int W>
__global__ __launch_bounds__(64) void k_interp_zgather(
    int n0, int n1, int n2, int nbx, int nby, int nzc, int zseg, int nseg, float bl2e,
    const int32_t *__restrict__ zstart, const uint32_t *__restrict__ perm,
    const uint32_t *__restrict__ word, CF3s frs, const float2 *__restrict__ grid,
    int64_t gstride, float2 *__restrict__ out, int64_t ostride) {
    constexpr int NX = ZB + W - 1;     // window columns per axis
    constexpr int NYP = (NX + 1) / 2;  // Y pairs of a window load
    static_assert(W >= 2 && NX <= 16 && ZC + W - 1 <= 16, "window exceeds the 16 K rows / slots");
    constexpr float kAScale = 16384.0f;  // 2^14 on wy
    __shared__ __align__(16) _Float16 atab[64 * AROW];
    __shared__ __align__(16) float wxt[NX * TROW];
    __shared__ __align__(16) float wzt[16 * TROW];
    __shared__ __align__(16) uint32_t pmt[64];
    __shared__ __align__(16) int oxt[64];  // x cell of the first tap, per row
    // one part (re or im) of a window half in the B layout: [X][g][n & 7][8]
    __shared__ __align__(16) _Float16 stg[NX * 4 * 8 * 8];

    int bx, by, seg;
    zs_block(xcd_remap(blockIdx.x, (int64_t)nbx * nby * nseg), nbx, nby, bx, by, seg);
    grid += (int64_t)blockIdx.y * gstride;
    out += (int64_t)blockIdx.y * ostride;
    const int lane = threadIdx.x, n = lane & 15, g = lane >> 4;
    const int64_t kb = ((int64_t)bx * nby + by) * nzc;
    const int c0 = seg * (zseg / ZC), c1 = min(c0 + zseg / ZC, nzc);
    int j = zstart[(kb + c0) * 16];
    const int jend = zstart[(kb + c1) * 16];
    if (j >= jend) return;  // no points in this block and segment

    {
        // K rows past the loaded Y pairs are never written: keep them zero
        // (times the zero A entries they meet)
        gf4 *s4 = reinterpret_cast<gf4 *>(stg);
        for (int i = lane; i < NX * 4 * 8; i += 64) s4[i] = gf4{0.f, 0.f, 0.f, 0.f};
    }
    gh8 bre[NX], bim[NX];  // the window (B operands), real and imaginary
#pragma unroll
    for (int X = 0; X < NX; ++X) {
        bre[X] = gh8{0, 0, 0, 0, 0, 0, 0, 0};
        bim[X] = gh8{0, 0, 0, 0, 0, 0, 0, 0};
    }
    int se0 = 0, se1 = 0;  // scale exponents of ring halves 0 and 1

    // z-run 8 cz .. 8 cz + 7 (periodic) of the window columns into ring half cz & 1
    auto load_half = [&](int cz) __attribute__((always_inline)) {
        const int h = cz & 1;
        const int zl = lane & 7, yp = lane >> 3;
        const int z = (ZC * cz + zl) % n2;
        const int ya = min(yp, NYP - 1);  // idle lanes read a real pair and drop it
        int y0 = ZB * by + 2 * ya, y1 = y0 + 1;
        if (y0 >= n1) y0 -= n1;
        if (y1 >= n1) y1 -= n1;
        const bool on0 = yp < NYP;
        const int o0 = y0 * n2 + z, o1 = y1 * n2 + z;
        const int64_t plane = (int64_t)n1 * n2;
        float2 v0[NX], v1[NX];
#pragma unroll
        for (int X = 0; X < NX; ++X) {
            int x = ZB * bx + X;
            if (x >= n0) x -= n0;
            // a uniform column base and 32-bit lane offsets (one address add
            // per load in the memory unit, none on the VALU)
            const char *col = reinterpret_cast<const char *>(grid + x * plane);
            v0[X] = *reinterpret_cast<const float2 *>(col + (uint32_t)o0 * 8u);
            v1[X] = *reinterpret_cast<const float2 *>(col + (uint32_t)o1 * 8u);
        }
        // (idle lanes and, for odd NX, the pair's second column Y = NX, which
        // meets only zero A entries, stage real grid values: finite grids
        // need no zeroing)
        float mx = 0.f;
#pragma unroll
        for (int X = 0; X < NX; ++X)
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v0[X].x), fabsf(v0[X].y)),
                                 fmaxf(fabsf(v1[X].x), fabsf(v1[X].y))));
        if (!on0) mx = 0.f;
        // the half's largest magnitude is below 2^(e - 126): scaled by
        // 2^(141 - e) every value is below 2^15
        const int s = 141 - wave_max9((__float_as_int(mx) >> 23) & 0xff);
        if (h)
            se1 = s;
        else
            se0 = s;
        uint32_t *sw = reinterpret_cast<uint32_t *>(stg);
#pragma unroll
        for (int part = 0; part < 2; ++part) {
            // lane (zl, yp): hi of Y = 2yp, 2yp + 1 at k = 2yp, lo at 16 + 2yp
            if (on0) {
#pragma unroll
                for (int X = 0; X < NX; ++X) {
                    const float a = __builtin_amdgcn_ldexpf(part ? v0[X].y : v0[X].x, s);
                    const float b = __builtin_amdgcn_ldexpf(part ? v1[X].y : v1[X].x, s);
                    const auto hi = __builtin_amdgcn_cvt_pkrtz(a, b);
                    uint32_t hb;
                    __builtin_memcpy(&hb, &hi, 4);
                    const uint32_t lb = split_lo(a, b, hb);
                    sw[((X * 4 + (yp >> 2)) * 8 + zl) * 4 + (yp & 3)] = hb;
                    sw[((X * 4 + 2 + (yp >> 2)) * 8 + zl) * 4 + (yp & 3)] = lb;
                }
            }
            if ((n >> 3) == h) {
                // read straight into the window registers of this half's
                // lanes (a plain load and masked merge costs a copy per
                // register); the reads are waited for here
                const uint32_t a = lds_addr(stg) + ((g * 8 + (n & 7)) * 8) * 2;
#pragma unroll
                for (int X = 0; X < NX; ++X) {
                    if (part)
                        ds_read_b128_into(bim[X], a, X * 4 * 8 * 8 * 2);
                    else
                        ds_read_b128_into(bre[X], a, X * 4 * 8 * 8 * 2);
                }
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            }
        }
    };

    int cw = INT32_MIN;  // the window's chunk: z-runs 8 cw and 8 cw + 8 loaded
    auto window_to = [&](int c) __attribute__((always_inline)) {
        if (c == cw) return;
        if (c != cw + 1) load_half(c);
        load_half(c + 1);
        cw = c;
    };

    // The loads of a batch's points: lanes [0, nA) take sorted index jA +
    // lane (chunk cA), lanes [oB, oB + nB) jB + lane - oB (chunk cB); the
    // other lanes read index 0, so every lane issues the same loads (the
    // batch after next is loading while a batch is built and swept).
    auto load_points = [&](const ZgBatch &b) __attribute__((always_inline)) {
        const bool inA = lane < b.nA, inB = lane >= b.oB && lane < b.oB + b.nB;
        const int jj = inA ? b.jA + lane : (inB ? b.jB + (lane - b.oB) : 0);
        ZgPoint q;
        q.wd = word[jj];
        q.fx = frs.p[0][jj];
        q.fy = frs.p[1][jj];
        q.fz = frs.p[2][jj];
        q.pj = perm[jj];
        return q;
    };

    auto prologue = [&](const ZgBatch &b, const ZgPoint &q) __attribute__((always_inline)) {
        {
            gf4 *wx4 = reinterpret_cast<gf4 *>(wxt);
            for (int i = lane; i < NX * TROW / 4; i += 64) wx4[i] = gf4{0.f, 0.f, 0.f, 0.f};
            gf4 *wz4 = reinterpret_cast<gf4 *>(wzt);
            for (int i = lane; i < 16 * TROW / 4; i += 64) wz4[i] = gf4{0.f, 0.f, 0.f, 0.f};
            gf4 *ar4 = reinterpret_cast<gf4 *>(atab + lane * AROW);
#pragma unroll
            for (int i = 0; i < 4; ++i) ar4[i] = gf4{0.f, 0.f, 0.f, 0.f};
        }
        const bool inA = lane < b.nA, inB = lane >= b.oB && lane < b.oB + b.nB;
        if (inA || inB) {
            const int cc = inA ? b.cA : b.cB;
            const uint32_t wd = q.wd;
            const float fx = q.fx, fy = q.fy, fz = q.fz;
            pmt[lane] = q.pj;
            const int ox = (int)((wd >> 23) & 7u), oy = (int)((wd >> 26) & 7u);
            oxt[lane] = ox;
            const int s0 = ZC * (cc & 1) + (int)(wd >> 29);  // ring slot of the first tap
            float *wxc = wxt + ox * TROW + lane;
            _Float16 *ar = atab + lane * AROW + oy;
            constexpr float ih = 2.0f / W;
#pragma unroll
            for (int a = 0; a < W; ++a) {
                const float ca = (float)a * ih;
                wxc[a * TROW] = zs_es(__builtin_fmaf(-fx, ih, ca), bl2e);
                const float vy = zs_es(__builtin_fmaf(-fy, ih, ca), bl2e) * kAScale;
                const auto hv = __builtin_amdgcn_cvt_pkrtz(vy, 0.f);
                ar[a] = hv[0];
                ar[16 + a] = (_Float16)(vy - (float)hv[0]);
                wzt[((s0 + a) & 15) * TROW + lane] = zs_es(__builtin_fmaf(-fz, ih, ca), bl2e);
            }
        }
    };

    // The x sums of one tile over the window columns [XS, XS + LEN), as
    // straight-line code: with no branch between columns the compiler
    // overlaps each column's MFMA chain and weight read with the next ones
    // (a branch per column left every step waiting on its own latencies).
    auto xrun = [&](auto XS, auto LEN, const gh8 &a1, const gh8 &a2, int t, float(&accr)[4],
                    float(&acci)[4]) __attribute__((always_inline)) {
        constexpr int xs = decltype(XS)::value, len = decltype(LEN)::value;
#pragma unroll
        for (int k = 0; k < len; ++k) {
            const int X = xs + k;
            gf4 cr = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, bre[X], gf4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            gf4 ci = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, bim[X], gf4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            cr = __builtin_amdgcn_mfma_f32_16x16x32_f16(a2, bre[X], cr, 0, 0, 0);
            ci = __builtin_amdgcn_mfma_f32_16x16x32_f16(a2, bim[X], ci, 0, 0, 0);
            const gf4 wv = *reinterpret_cast<const gf4 *>(wxt + X * TROW + 16 * t + 4 * g);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                accr[i] = __builtin_fmaf(wv[i], cr[i], accr[i]);
                acci[i] = __builtin_fmaf(wv[i], ci[i], acci[i]);
            }
        }
    };
    // a tile's columns fit a window of XL = w + 2 (x cells of its first and
    // last rows at most 2 apart, the usual case) or take all NX
    constexpr int XL = W + 2;
    using XLc = std::integral_constant<int, XL>;

    // tiles [t0, t1) of the batch; rows [pb, pe) hold points. The reduction
    // of tile t - 1 sits in the basic block of tile t's MFMA chain, so that
    // its VALU and DPP work fills the matrix-core shadow (measured 1-1.5 %
    // faster than reducing each tile after its own chain); its store follows.
    auto tiles = [&](int t0, int t1, int pb, int pe) __attribute__((always_inline)) {
        const int esc = -((n >> 3) ? se1 : se0) - 14;
        const bool b2 = n & 4, b1 = n & 2, b0 = n & 1;
        // reduce-scatter over each half row of 8 lanes (one slot scale),
        // leaving lane n with value n & 7 (point 4g + ((n & 7) >> 1), part
        // n & 1); unscale; add the two halves
        auto reduce = [&](const float (&v)[8]) __attribute__((always_inline)) {
            float u[4], w2[2];
#pragma unroll
            for (int k = 0; k < 4; ++k)
                u[k] = (b2 ? v[k + 4] : v[k]) + dpp_f<kDppRowHalfMirror>(b2 ? v[k] : v[k + 4]);
#pragma unroll
            for (int k = 0; k < 2; ++k)
                w2[k] = (b1 ? u[k + 2] : u[k]) + dpp_f<kDppQuadMirror>(b1 ? u[k] : u[k + 2]);
            float r = (b0 ? w2[1] : w2[0]) + dpp_f<kDppQuadSwap>(b0 ? w2[0] : w2[1]);
            r = __builtin_amdgcn_ldexpf(r, esc);
            return r + dpp_f<kDppRowRor8>(r);
        };
        float pv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        int pq = -1;  // tile whose products pv holds
        // (stores of the results straight from the tile measured 0.15 ms
        // faster than staging a batch's results in LDS for one store)
        auto store = [&](float r, int q) __attribute__((always_inline)) {
            const int p = 16 * q + 4 * g + ((n & 7) >> 1);
            const float o = dpp_f<kDppQuadSwap>(r);
            if (n < 8 && (n & 1) == 0 && p >= pb && p < pe)
                out[pmt[p]] = make_float2(r, o);
        };
        for (int t = t0; t < t1; ++t) {
            const int xlo = __builtin_amdgcn_readfirstlane(oxt[max(16 * t, pb)]);
            const int xhi = __builtin_amdgcn_readfirstlane(oxt[min(16 * t + 16, pe) - 1]) + W;
            const _Float16 *ar = atab + (16 * t + n) * AROW + 8 * (g & 1);
            const gh8 a1 = *reinterpret_cast<const gh8 *>(ar);
            gh8 a2 = *reinterpret_cast<const gh8 *>(ar + 16);
            if (g >= 2) a2 = gh8{0, 0, 0, 0, 0, 0, 0, 0};
            float accr[4] = {0.f, 0.f, 0.f, 0.f}, acci[4] = {0.f, 0.f, 0.f, 0.f};
            float r = 0.f;
            auto body = [&](auto XS, auto LEN) __attribute__((always_inline)) {
                r = reduce(pv);
                xrun(XS, LEN, a1, a2, t, accr, acci);
            };
            if (xhi - xlo <= XL) {
                const int xs = min(xlo, NX - XL);
                auto pick = [&](auto... I) __attribute__((always_inline)) {
                    ((xs == decltype(I)::value ? body(I, XLc{}) : void()), ...);
                };
                static_assert(NX - XL == 5, "six window offsets");
                pick(std::integral_constant<int, 0>{}, std::integral_constant<int, 1>{},
                     std::integral_constant<int, 2>{}, std::integral_constant<int, 3>{},
                     std::integral_constant<int, 4>{}, std::integral_constant<int, 5>{});
            } else {
                body(std::integral_constant<int, 0>{}, std::integral_constant<int, NX>{});
            }
            if (pq >= 0) store(r, pq);
            const gf4 wz = *reinterpret_cast<const gf4 *>(wzt + n * TROW + 16 * t + 4 * g);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                pv[2 * i] = accr[i] * wz[i];
                pv[2 * i + 1] = acci[i] * wz[i];
            }
            pq = t;
        }
        if (pq >= 0) store(reduce(pv), pq);
    };

    // the next batch from the cursor (c: chunk of sorted index j, cend its end)
    int c = c0, cend = zstart[(kb + c0 + 1) * 16];
    auto next_batch = [&]() __attribute__((always_inline)) {
        ZgBatch b{0, 0, 0, 64, 0, 0, 0};
        if (j >= jend) return b;
        while (j >= cend) {
            ++c;
            cend = zstart[(kb + c + 1) * 16];
        }
        b.cA = b.cB = c;
        b.jA = j;
        b.nA = min(64, cend - j);
        j += b.nA;
        b.oB = (b.nA + 15) & ~15;
        if (b.oB < 64 && j < jend) {
            while (j >= cend) {
                ++c;
                cend = zstart[(kb + c + 1) * 16];
            }
            b.cB = c;
            b.jB = j;
            b.nB = min(64 - b.oB, cend - j);
            j += b.nB;
        }
        return b;
    };

    // Memory waits count loads and stores together, in issue order, so the
    // window loads of the next batch go out before this batch's stores:
    // waiting for them then does not wait for the scattered stores, which
    // complete while the next batch is built and swept.
    ZgBatch cur = next_batch();
    ZgPoint pc = load_points(cur);
    for (;;) {
        const ZgBatch nxt = next_batch();
        const ZgPoint pn = load_points(nxt);
        // compiler-only fences keep the tables' program order (written as
        // scalars, read as vectors; the wave's LDS operations complete in
        // issue order, so no wait is needed)
        asm volatile("" ::: "memory");
        prologue(cur, pc);
        asm volatile("" ::: "memory");
        // parts A and B through one copy of the window and tile code
#pragma nounroll
        for (int part = 0; part < 2; ++part) {
            if (part == 1 && cur.nB == 0) break;
            const int p0 = part ? cur.oB : 0, p1 = part ? cur.oB + cur.nB : cur.nA;
            window_to(part ? cur.cB : cur.cA);
            tiles(p0 >> 4, (p1 + 15) >> 4, p0, p1);
        }
        if (nxt.nA == 0) break;
        cur = nxt;
        pc = pn;
    }
}

struct GArgs {
    const mn_bins *g;
    float beta;
    int zseg;
    const int32_t *zstart;
    const uint32_t *perm;
    const uint32_t *word;
    CF3s frs;
    const float2 *grid;
    float2 *out;
    int64_t B, P;
    hipStream_t s;
};

template <int DIM, int W>
struct GLaunch {
    static int run(const GArgs &a) {
        if constexpr (DIM != 3 || W > ZB) {
            set_error("zgather: unsupported dim/width");
            return MN_EINVAL;
        } else {
            const int n0 = (int)a.g->n[0], n1 = (int)a.g->n[1], n2 = (int)a.g->n[2];
            const int nbx = n0 / ZB, nby = n1 / ZB, nseg = (n2 + a.zseg - 1) / a.zseg;
            const int nzc = (n2 + ZC - 1) / ZC;
            const int64_t nw = (int64_t)nbx * nby * nseg;
            const float bl2e = (float)(a.beta * 1.4426950408889634);
            const int64_t gs = (int64_t)n0 * n1 * n2;
            const dim3 gridd((unsigned)nw, (unsigned)a.B);
            k_interp_zgather<W><<<gridd, 64, 0, a.s>>>(n0, n1, n2, nbx, nby, nzc, a.zseg, nseg,
                                                       bl2e, a.zstart, a.perm, a.word, a.frs,
                                                       a.grid, gs, a.out, a.P);
            MN_LAUNCH_CHECK("interp_zgather");
            return MN_OK;
        }
    }
};

}  // namespace
}  // namespace mn

using namespace mn;

extern "C" {

int mn_interp_zgather(const mn_bins *g, float beta, int64_t P, int64_t B, int zseg,
                      const int32_t *zstart, const uint32_t *perm, const uint32_t *sorted_word,
                      const float *const frs[3], const void *grids, void *outs,
                      mn_stream_t stream) {
    clear_error();
    int rc = zsweep_check(g);
    if (rc) return rc;
    MN_REQUIRE(P >= 1 && P < (int64_t(1) << 31), "zgather: P must be in [1, 2^31)");
    MN_REQUIRE(B >= 1 && B < 65536, "zgather: B must be in [1, 65535]");
    MN_REQUIRE(zseg >= ZC && zseg % ZC == 0, "zgather: zseg must be a positive multiple of 8");
    MN_REQUIRE(zstart && perm && sorted_word && grids && outs, "zgather: NULL pointer");
    GArgs a{};
    for (int d = 0; d < 3; ++d) {
        MN_REQUIRE(frs[d], "zgather: NULL sorted fraction pointer");
        a.frs.p[d] = frs[d];
    }
    a.g = g;
    a.beta = beta;
    a.zseg = zseg;
    a.zstart = zstart;
    a.perm = perm;
    a.word = sorted_word;
    a.grid = static_cast<const float2 *>(grids);
    a.out = static_cast<float2 *>(outs);
    a.B = B;
    a.P = P;
    a.s = as_stream(stream);
    return select_dim_w<GLaunch>(3, g->w, a);
}

}  // extern "C"
