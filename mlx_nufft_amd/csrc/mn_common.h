// Shared helpers of the HIP sources: error state, argument checks, the ES
// kernel, periodic wrap, and the XCD-aware workgroup remap.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/mlx_nufft_amd.h"

namespace mn {

// ---- error state (one message per host thread) ---------------------------
void set_error(const std::string &msg);
void clear_error();

#define MN_REQUIRE(cond, msg)                 \
    do {                                      \
        if (!(cond)) {                        \
            ::mn::set_error(msg);             \
            return MN_EINVAL;                 \
        }                                     \
    } while (0)

#define MN_HIP_CHECK(expr)                                                    \
    do {                                                                      \
        hipError_t _e = (expr);                                               \
        if (_e != hipSuccess) {                                               \
            ::mn::set_error(std::string(#expr) + ": " + hipGetErrorString(_e)); \
            return MN_ERUNTIME;                                               \
        }                                                                     \
    } while (0)

// Check a kernel launch (launch-configuration errors surface here).
#define MN_LAUNCH_CHECK(what)                                                   \
    do {                                                                        \
        hipError_t _e = hipGetLastError();                                      \
        if (_e != hipSuccess) {                                                 \
            ::mn::set_error(std::string(what) + " launch: " + hipGetErrorString(_e)); \
            return MN_ERUNTIME;                                                 \
        }                                                                       \
    } while (0)

inline hipStream_t as_stream(mn_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Validate a bin geometry; returns MN_OK or sets the error and MN_EINVAL.
int check_bins(const mn_bins *g);

inline int64_t nbins_total(const mn_bins *g) {
    int64_t t = 1;
    for (int d = 0; d < g->dim; ++d) t *= g->nb[d];
    return t;
}

inline int64_t tile_cells(const mn_bins *g) {
    int64_t t = 1;
    for (int d = 0; d < g->dim; ++d) t *= (int64_t)g->m[d] + g->w - 1;
    return t;
}

// LDS bytes available to one workgroup on the current device.
int max_lds_per_block();

// Releases the cached twiddle tables of the fp64 line FFTs (mn_fftl.hip).
void fftl_cache_clear();

// Zero device memory with a fill kernel (usable under graph capture).
int fill_zero(void *ptr, int64_t bytes, hipStream_t s);

// Exclusive prefix sum of n uint32 values in place; `partials` must hold
// scan_partials_elems(n) uint32 of scratch. Returns MN_OK or an error.
int64_t scan_partials_elems(int64_t n);
int scan_exclusive_u32(uint32_t *data, int64_t n, uint32_t *partials, hipStream_t s);

// starts[k] = first index of the sorted keys whose key & kmask is >= k, for
// k in [0, K] (K + 1 entries); keys must be < K after masking.
int key_starts(const uint32_t *sorted_key, int64_t P, int64_t K, uint32_t kmask, int32_t *starts,
               hipStream_t s);

constexpr int kMaxW = 16;
constexpr double kTwoPi = 6.283185307179586;  // fl64(2*pi)

// Kernel geometry passed by value to the device.
struct Geom {
    int dim;
    int w;
    int n[3];   // grid size per dim (1 for unused dims)
    int m[3];   // bin size
    int nb[3];  // bins per dim
    int p[3];   // padded tile size m + w - 1 (1 for unused dims)
};

inline Geom make_geom(const mn_bins *g) {
    Geom k;
    k.dim = g->dim;
    k.w = g->w;
    for (int d = 0; d < 3; ++d) {
        bool used = d < g->dim;
        k.n[d] = used ? (int)g->n[d] : 1;
        k.m[d] = used ? g->m[d] : 1;
        k.nb[d] = used ? g->nb[d] : 1;
        k.p[d] = used ? g->m[d] + g->w - 1 : 1;
    }
    return k;
}

// ---- device helpers -------------------------------------------------------

// ES kernel psi(d) = exp(beta*(sqrt(1 - (2d/w)^2) - 1)) on |d| <= w/2.
// Written as 2^(beta*log2(e)*(sqrt(t)-1)) on the hardware v_sqrt_f32 and
// v_exp_f32 (about 1 ulp each); bl2e = beta*log2(e), inv_hw = 2/w. The exp2
// argument lies in [-bl2e, 0] (bl2e <= 0.97*pi*log2(e)*16, about 71), so no
// denormal input or result arises and the libm wrappers' range fix-ups
// (some 20 extra instructions per weight) are not needed. Callers mask taps
// with |d| > w/2 themselves (t is clamped to 0 there, giving e^-beta).
__device__ __forceinline__ float es_weight(float d, float bl2e, float inv_hw) {
    const float z = d * inv_hw;
    const float t = fmaxf(1.0f - z * z, 0.0f);
    return __builtin_amdgcn_exp2f(bl2e * (__builtin_amdgcn_sqrtf(t) - 1.0f));
}

// The same kernel with the exponent written -bl2e z^2 / (1 + sqrt(1 - z^2)),
// equal to bl2e (sqrt(1 - z^2) - 1) in exact arithmetic but free of its
// cancellation near z = 0, where the fp32 rounding of the square root would
// enter the weight multiplied by beta (about 1e-6 relative at beta = 16).
// Used where the grid's error is amplified afterwards (the type-3 spread,
// whose inner grid is deconvolved twice).
__device__ __forceinline__ float es_weight_stable(float d, float bl2e, float inv_hw) {
    const float z = d * inv_hw;
    const float z2 = z * z;
    const float t = fmaxf(1.0f - z2, 0.0f);
    return __builtin_amdgcn_exp2f(-bl2e * z2 *
                                  __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_sqrtf(t)));
}

// The same kernel at the scaled distance z = 2d/w: the exp2 argument
// bl2e*(sqrt(t) - 1) is one fma. For |z| > 1 it returns e^-beta (t clamped
// to 0); callers mask those taps.
__device__ __forceinline__ float es_weight_z(float z, float bl2e) {
    const float t = fmaxf(fmaf(-z, z, 1.0f), 0.0f);
    return __builtin_amdgcn_exp2f(fmaf(bl2e, __builtin_amdgcn_sqrtf(t), -bl2e));
}

// Map a cell index that is at most one period outside [0, n) back into it.
__device__ __forceinline__ int wrap1(int i, int n) {
    i += (i < 0) ? n : 0;
    i -= (i >= n) ? n : 0;
    return i;
}

// True modulo into [0, n) for any int.
__device__ __forceinline__ int pmod(int i, int n) {
    int r = i % n;
    return r < 0 ? r + n : r;
}

// Workgroups are dispatched round-robin over the 8 XCDs (blockIdx % 8).
// Remap so that XCD k receives one contiguous run of work items, which keeps
// neighbouring bins (and the grid lines their tiles share) in one L2.
__device__ __forceinline__ int64_t xcd_remap(int64_t bid, int64_t nblk) {
    constexpr int64_t NX = 8;
    if (nblk < NX) return bid;
    int64_t q = nblk / NX, r = nblk % NX;
    int64_t x = bid % NX, slot = bid / NX;
    return x * q + (x < r ? x : r) + slot;
}

// Sorted per-point arrays, by value into kernels.
struct CI3s { const int32_t *p[3]; };
struct CF3s { const float *p[3]; };

// ---- z-sweep point word ----------------------------------------------------
// The 3D owner-computes spread sorts one 32-bit word per point:
//   bits  0-22  key = ((bx*nby + by)*nzc + zc)*16 + rank(cx, cy) (sorted on)
//   bits 23-25  x cell of the first tap within its 8-column block
//   bits 26-28  y cell likewise
//   bits 29-31  z cell of the first tap within its 8-cell z-chunk
// where (bx, by) is the 8x8 column block of the first tap (x, y), zc = z / 8
// its z-chunk (nzc = ceil(n2 / 8) chunks), and (cx, cy) the reach codes of
// the first tap along x and y (zs_reach). Inside a (block, chunk) the order
// of the points does not matter to the spread (its z-window spans the whole
// chunk), so the key stops at the chunk and the low bits group the points
// by how their footprint meets the blocks.
constexpr int kZsBlock = 8;
constexpr int kZsChunk = 8;
constexpr int kZsKeyBits = 23;
constexpr uint32_t kZsKeyMask = (1u << kZsKeyBits) - 1u;

// Reach code of a first tap at cell o (0..7) of its block for width w:
// 0 when the footprint stays inside the block, else it reaches the next
// block and is 1 when it also covers the lower half (cells 0..3) of its own
// block, 3 when it also covers the upper half of the next block, 2 when
// neither.
__host__ __device__ __forceinline__ int zs_reach(int o, int w) {
    if (o + w - 1 < kZsBlock) return 0;
    if (o <= 3) return 1;
    return (o + w - 1 >= kZsBlock + 4) ? 3 : 2;
}

// Rank of the class (cx, cy) in the key. Classes that reach along x (cx >
// 0) take ranks 3..14 and those that reach along y (cy > 0) ranks 0..11, so
// the points a block receives from each neighbour are one key range:
// own block [0, 16), -x neighbour [3, 15), -y neighbour [0, 12), -xy
// neighbour [3, 12).
__host__ __device__ __forceinline__ int zs_rank(int cx, int cy) {
    if (cx == 0) return cy == 0 ? 15 : cy - 1;
    return cy == 0 ? 11 + cx : 3 * cx + cy - 1;
}

__device__ __forceinline__ uint32_t zs_word(int x, int y, int z, int n1, int nzc, int w) {
    const int lx = x & (kZsBlock - 1), ly = y & (kZsBlock - 1), lz = z & (kZsChunk - 1);
    const uint32_t blk = (uint32_t)((x / kZsBlock) * (n1 / kZsBlock) + y / kZsBlock);
    const uint32_t key = (blk * (uint32_t)nzc + (uint32_t)(z / kZsChunk)) * 16u +
                         (uint32_t)zs_rank(zs_reach(lx, w), zs_reach(ly, w));
    return key | ((uint32_t)lx << 23) | ((uint32_t)ly << 26) | ((uint32_t)lz << 29);
}

// The z-gather interpolation sorts the same word with a key that orders
// the points of a (block, chunk) by the x cell of their first tap instead of
// by class: key = ((bx*nby + by)*nzc + zc)*16 + 2*lx, so the key space, the
// chunk starts (zstart at multiples of 16) and the word's upper bits are
// those of zs_word.
__device__ __forceinline__ uint32_t zg_word(int x, int y, int z, int n1, int nzc) {
    const int lx = x & (kZsBlock - 1), ly = y & (kZsBlock - 1), lz = z & (kZsChunk - 1);
    const uint32_t blk = (uint32_t)((x / kZsBlock) * (n1 / kZsBlock) + y / kZsBlock);
    const uint32_t key = (blk * (uint32_t)nzc + (uint32_t)(z / kZsChunk)) * 16u + 2u * (uint32_t)lx;
    return key | ((uint32_t)lx << 23) | ((uint32_t)ly << 26) | ((uint32_t)lz << 29);
}

// Validate a z-sweep geometry (3D, 2 <= w <= 8, n0 and n1 multiples of 8 and
// >= 16, key space within kZsKeyBits); number of keys
// K = nbx*nby*ceil(n2/8)*16.
int zsweep_check(const mn_bins *g);
int64_t zsweep_nkeys(const mn_bins *g);

// ---- y-sweep point word (2D) ---------------------------------------------
// The 2D owner-computes spread sorts one 32-bit word per point:
//   bits  0-25  key = (bx*n1 + y)*2 + reach (sorted on)
//   bits 26-31  x cell of the first tap within its 64-column block
// where bx is the 64-column block of the first tap x, y its cell, and reach
// says whether the footprint crosses into the next block.
constexpr int kYsBlock = 64;
constexpr int kYsKeyBits = 26;
constexpr uint32_t kYsKeyMask = (1u << kYsKeyBits) - 1u;

__device__ __forceinline__ uint32_t ys_word(int x, int y, int n1, int w) {
    const int lx = x & (kYsBlock - 1);
    const uint32_t reach = (lx + w - 1 >= kYsBlock) ? 1u : 0u;
    const uint32_t key = ((uint32_t)(x / kYsBlock) * (uint32_t)n1 + (uint32_t)y) * 2u + reach;
    return key | ((uint32_t)lx << kYsKeyBits);
}

// Validate a y-sweep geometry (2D, 2 <= w <= 8, n0 a multiple of 64 and
// >= 128, key space within kYsKeyBits); number of keys K = (n0/64)*n1*2.
int ysweep_check(const mn_bins *g);
int64_t ysweep_nkeys(const mn_bins *g);

// ---- y-window MFMA sweep point word (2D) ------------------------------------
// The 2D spread on the matrix cores (mn_ymfma.hip) sorts one 32-bit word per
// point:
//   bits  0-24  key = (bx*nyc + yc)*2 + reach (sorted on)
//   bits 25-28  x cell of the first tap within its 16-column block
//   bits 29-31  y cell of the first tap within its 8-cell y-chunk
// where bx is the 16-column block of the first tap x, yc = y / 8 its y-chunk
// (nyc = n1 / 8 chunks) and reach says whether the footprint crosses into
// the next block. Inside a (block, chunk) the order of the points does not
// matter to the spread (its y-window spans the whole chunk).
constexpr int kYmBlock = 16;
constexpr int kYmChunk = 8;
constexpr int kYmKeyBits = 25;
constexpr uint32_t kYmKeyMask = (1u << kYmKeyBits) - 1u;

__device__ __forceinline__ uint32_t ym_word(int x, int y, int nyc, int w) {
    const int lx = x & (kYmBlock - 1), ly = y & (kYmChunk - 1);
    const uint32_t reach = (lx + w - 1 >= kYmBlock) ? 1u : 0u;
    const uint32_t key =
        ((uint32_t)(x / kYmBlock) * (uint32_t)nyc + (uint32_t)(y / kYmChunk)) * 2u + reach;
    return key | ((uint32_t)lx << kYmKeyBits) | ((uint32_t)ly << 29);
}

// Validate a y-window MFMA sweep geometry (2D, 2 <= w <= 8, n0 a multiple
// of 16 and >= 32, n1 a multiple of 8 and >= 16, key space within
// kYmKeyBits); number of keys K = (n0/16)*(n1/8)*2.
int ymfma_check(const mn_bins *g);
int64_t ymfma_nkeys(const mn_bins *g);

// Validate the point/subproblem arguments shared by spread and interp.
int check_points(const mn_bins *g, int64_t P, int64_t nsub, const int32_t *info,
                 const uint32_t *perm, const int32_t *const i1s[3], const float *const frs[3],
                 CI3s *ci, CF3s *cf);

// Pick the (DIM, W) instantiation of a launcher template at run time.
template <template <int, int> class L, typename A, int DIM, int W>
int select_w(int w, const A &a) {
    if constexpr (W > kMaxW) {
        set_error("kernel width out of range");
        return MN_EINVAL;
    } else {
        if (w == W) return L<DIM, W>::run(a);
        return select_w<L, A, DIM, W + 1>(w, a);
    }
}

template <template <int, int> class L, typename A>
int select_dim_w(int dim, int w, const A &a) {
    switch (dim) {
        case 1: return select_w<L, A, 1, 2>(w, a);
        case 2: return select_w<L, A, 2, 2>(w, a);
        case 3: return select_w<L, A, 3, 2>(w, a);
    }
    set_error("dim must be 1, 2 or 3");
    return MN_EINVAL;
}

}  // namespace mn
