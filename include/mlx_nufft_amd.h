/*
 * mlx_nufft_amd.h -- C-ABI of the MI355X NUFFT engine (libmlxnufft_amd.so).
 *
 * Every entry point is asynchronous on the HIP stream it is given (the
 * caller's stream; from PyTorch, torch.cuda.current_stream().cuda_stream),
 * takes plain device pointers and sizes, and returns an int status:
 *   MN_OK (0), MN_EINVAL (-1, bad argument), MN_ERUNTIME (-2, HIP/rocFFT
 *   failure), MN_ENOTIMPL (-3, unsupported combination).
 * On a non-zero status, mn_last_error() returns a message for the calling
 * thread. The library owns no caller data; it keeps only mutex-guarded
 * caches: rocFFT plans (plus their work buffers) and the twiddle tables of
 * the fp64 line FFTs, both released by mn_fft_cache_clear.
 *
 * Complex data are interleaved complex64 (float re, float im) -- the
 * layout of numpy/torch complex64. Grids are C-ordered (last dim fastest).
 *
 * Citations "ref:" name the reference (mlx-nufft) code each entry point
 * replaces; the reference's kernels are Metal source strings built per plan
 * and launched through mx.fast.metal_kernel, so the citations point at
 * those builders and launches.
 */
#ifndef MLX_NUFFT_AMD_H
#define MLX_NUFFT_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MN_OK 0
#define MN_EINVAL (-1)
#define MN_ERUNTIME (-2)
#define MN_ENOTIMPL (-3)

typedef void *mn_stream_t; /* a hipStream_t; NULL = the default stream */

/*
 * Fine-grid bin geometry shared by setpts, sort, spread and interp.
 * dim in {1,2,3}; w = ES kernel width (2..16); n[d] = fine-grid size along
 * dim d (1 for d >= dim); m[d] = bin size (cells) along d; nb[d] = number
 * of bins along d = ceil(n[d]/m[d]). A point with cell index i1 (leftmost
 * tap) lies in bin b[d] = ((i1[d] + w/2) mod n[d]) / m[d]; its bin key is
 * the row-major index of b over nb. The padded tile of a bin has
 * p[d] = m[d] + w - 1 cells and origin b[d]*m[d] - w/2.
 * ref: nd.py:282-296 (_od_tile_dims), nd.py:298-320 (_od_prepare key).
 */
typedef struct mn_bins {
    int32_t dim;
    int32_t w;
    int64_t n[3];
    int32_t m[3];
    int32_t nb[3];
} mn_bins;

/* Message of the last failed call on this thread ("" if none). */
const char *mn_last_error(void);
/* ABI version (major*10000 + minor*100 + patch). */
int mn_version(void);
/* LDS bytes one workgroup may use on the current device (bounds the bin
 * tiles: prod_d (m[d] + w - 1) cells of 16 bytes for the tile spread, which
 * accumulates in fp64, and of 8 bytes for interp). */
int mn_device_lds_bytes(void);

/*
 * Type-1/2 point setup ("crit64"): per point and dim, r = x mod 2pi with
 * numpy's np.mod semantics, xi = r / h (h = 2pi/n[d], fp64 division),
 * i1 = ceil(xi - w/2) (int32), fr = (float)(xi - i1), and the bin key.
 * prec64 = 1 reproduces the fp64 path bit for bit; prec64 = 0 the "fp32"
 * path (r and h rounded to fp32, fp32 divide).
 * ref: nd.py:152-165 (_compute_cells), nd.py:43-91 + nd.py:191-222
 * (df64 GPU re-point), nd.py:308-313 (bin key).
 */
int mn_setpts_t12(const mn_bins *g, int64_t P, const double *const x[3],
                  int prec64, int32_t *const i1[3], float *const fr[3],
                  uint32_t *key, mn_stream_t stream);

/*
 * Stable LSD radix sort of P uint32 keys (key_bits significant bits):
 * perm_out = argsort(key_in, stable), key_out = key_in[perm_out].
 * ws must hold mn_sort_workspace_bytes(P) bytes of device memory.
 * ref: nd.py:314 (np.argsort(key, kind="stable")), nd.py:338 (mx.argsort),
 * nd.py:175 (lateral sort), gpu_t3.py:490-492, gpu_t3.py:546.
 */
int64_t mn_sort_workspace_bytes(int64_t P);
int mn_sort_keys(int64_t P, int key_bits, const uint32_t *key_in,
                 uint32_t *key_out, uint32_t *perm_out, void *ws,
                 int64_t ws_bytes, mn_stream_t stream);

/*
 * The same stable sort carrying ncols (<= MN_SORT_MAX_COLS) 32-bit payload
 * columns: cols_out[c][r] = cols_in[c][perm_out[r]]. Only the low key_bits
 * bits of a key are sorted on; higher bits travel with the key unchanged.
 * Moving the per-point data through the radix passes replaces a gather by
 * perm (one cache line per 4-byte element) with coalesced tile writes.
 * ws must hold mn_sort_pairs_workspace_bytes(P, ncols) bytes.
 * ref: nd.py:314-318 (argsort, then take of i1/fr by perm), nd.py:338-340.
 */
#define MN_SORT_MAX_COLS 8
int64_t mn_sort_pairs_workspace_bytes(int64_t P, int ncols);
int mn_sort_pairs(int64_t P, int key_bits, const uint32_t *key_in, uint32_t *key_out,
                  uint32_t *perm_out, int ncols, const uint32_t *const *cols_in,
                  uint32_t *const *cols_out, void *ws, int64_t ws_bytes,
                  mn_stream_t stream);

/*
 * mn_sort_pairs without a workspace argument: it allocates nothing and
 * calls no allocating routine; its workspace is a 96 MiB device array in
 * the library (one per GPU, held until the process ends). No counterpart
 * in the reference: it is for callers that cannot allocate (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Limit: mn_sort_pairs_workspace_bytes(P, ncols) <= 96 MiB, about 1.2e7
 * points with no payload column and 5.0e6 with 3; larger sorts return
 * MN_EINVAL with a message. Every call on one GPU shares that GPU's array,
 * so calls that overlap on one GPU (other streams, other host threads) race;
 * calls on one stream are ordered and safe. Results are bit-identical to
 * mn_sort_pairs.
 */
int mn_sort_pairs_noalloc(int64_t P, int key_bits, const uint32_t *key_in, uint32_t *key_out,
                          uint32_t *perm_out, int ncols, const uint32_t *const *cols_in,
                          uint32_t *const *cols_out, mn_stream_t stream);

/*
 * Gather per-point arrays into sorted order: out[j] = in[perm[j]] for i1
 * and fr of each dim, and for an optional complex64 array (extra_in may
 * be NULL). ref: nd.py:316-318, nd.py:339-340, gpu_t3.py:496-501.
 */
int mn_gather_points(int dim, int64_t P, const uint32_t *perm,
                     const int32_t *const i1_in[3], const float *const fr_in[3],
                     int32_t *const i1_out[3], float *const fr_out[3],
                     const void *extra_in, void *extra_out, mn_stream_t stream);

/*
 * Subproblem table from the sorted bin keys: every non-empty bin is split
 * into chunks of at most msub points; sub_info receives 3 int32 per
 * subproblem (bin key, first sorted index, count), ordered by bin. The
 * table needs room for max_sub = nbins + P/msub + 1 rows. *nsub_out is
 * written on the host after the stream is synchronised (this call blocks).
 * ws must hold mn_subproblem_workspace_bytes(g) bytes.
 * ref: nd.py:347-372 (_od_finish), nd.py:341 (the reference's P-length
 * host sync, replaced here by one 8-byte read-back).
 */
int64_t mn_subproblem_workspace_bytes(const mn_bins *g);
int mn_build_subproblems(const mn_bins *g, int64_t P, const uint32_t *sorted_key,
                         int32_t msub, int32_t *sub_info, int64_t max_sub,
                         int64_t *nsub_out, void *ws, int64_t ws_bytes,
                         mn_stream_t stream);

/*
 * Spread (type-1 core): grid[cell] = sum_j c_j * prod_d psi(cell_d - x_j,d)
 * over the periodic fine grid, psi(d) = exp(beta*(sqrt(1-(2d/w)^2)-1)).
 * Points are read in sorted order (i1s/frs) and their strengths gathered
 * as c[perm[j]] (c in caller order); if pre != NULL the strength is
 * multiplied by pre[j] (sorted order; the type-3 prephase). One workgroup
 * per subproblem accumulates its padded tile in LDS and flushes it with
 * fp32 global atomics. grid (prod n complex64) is overwritten.
 * ref: nd.py:492-579 + nd.py:590-601 (OD spread), nd.py:437-490 (GM
 * spread), gpu_t3.py:565-591 + gpu_t3.py:1302-1311 (type-3 spread).
 */
int mn_spread(const mn_bins *g, float beta, int64_t P, int64_t nsub,
              const int32_t *sub_info, const uint32_t *perm,
              const int32_t *const i1s[3], const float *const frs[3],
              const void *c, const void *pre, void *grid, mn_stream_t stream);

/*
 * As mn_spread, but adds into the existing grid contents (no zero-fill):
 * lets a caller accumulate several point sets into one grid, or zero the
 * grid itself (mn_fill_zero) and time the spread kernel on its own.
 * ref: nd.py:590-601 (spread launch with init_value=0 split in two).
 */
int mn_spread_accumulate(const mn_bins *g, float beta, int64_t P, int64_t nsub,
                         const int32_t *sub_info, const uint32_t *perm,
                         const int32_t *const i1s[3], const float *const frs[3],
                         const void *c, const void *pre, void *grid,
                         mn_stream_t stream);

/*
 * mn_spread into a complex128 grid, with the strength times its prephase
 * and every strength x weight product formed in fp64 and the tiles flushed
 * with fp64 atomics (ES weights stay fp32): the type-3 source spread. Its
 * grid is deconvolved by 1/phihat at the band edges and again by
 * 1/phihat(theta) at the targets, which amplifies white rounding noise in
 * the grid about 20x (fp32 tap products and flush add ~1e-5 relative error
 * at 1e6 x 1e6 points, eps 1e-5); the fp32 weight error, a smooth function
 * of the fraction, is not amplified. ref: gpu_t3.py:565-591.
 */
int mn_spread_c128(const mn_bins *g, float beta, int64_t P, int64_t nsub,
                   const int32_t *sub_info, const uint32_t *perm,
                   const int32_t *const i1s[3], const float *const frs[3], const void *c,
                   const void *pre, void *grid, mn_stream_t stream);

/*
 * The same fp64 spread into a complex128 3D grid, owner-computes: one
 * workgroup per bin sums the taps that land in its bin from the points of
 * every bin whose footprints reach it, in an fp64 LDS tile of just the bin,
 * and stores the bin with plain writes. Every cell of the grid is written
 * once: no zero fill, no global atomics. Points are sorted by bin (the key
 * of mn_t3_setpts_src on the same geometry), bin_start[b] is the first
 * sorted point of bin b (mn_bin_starts, nbins + 1 entries), pre is in
 * sorted order (may be NULL). Bins need 16 * m0*m1*m2 bytes of LDS and,
 * along a dim with more than one bin, m >= w - 1.
 * ref: gpu_t3.py:565-591 (t3spread), nd.py:492-579 (the output-driven spread
 * idea).
 */
int mn_spread_owner_c128(const mn_bins *g, float beta, int64_t P, const int32_t *bin_start,
                         const uint32_t *perm, const int32_t *const i1s[3],
                         const float *const frs[3], const void *c, const void *pre, void *grid,
                         mn_stream_t stream);

/*
 * Owner-computes 3D spread ("z-sweep"), the fast path for 3D type-1 grids
 * with n0, n1 multiples of 8 (>= 16), n2 >= 8, w <= 8 and at most 2^23 sort
 * keys ((n0/8)(n1/8) ceil(n2/8) 16: 512^3 or 1024^2 x 256). Each wavefront
 * owns an 8x8 (x, y) column block over a z-segment of zseg cells (a positive
 * multiple of 8), sweeps it upwards in 8-cell z-chunks with the z-window of
 * each 4x4 quadrant in matrix-core accumulators, and stores every grid cell
 * exactly once (no atomics; grid is fully overwritten).
 * g: dim 3, w, n (m and nb are not used).
 *
 * Point word (one uint32 per point, from mn_zsweep_setpts):
 *   bits  0-22  key = ((bx*(n1/8) + by)*ceil(n2/8) + z/8)*16 + rank, where
 *               (bx, by) is the 8x8 block of the first tap, z its cell, and
 *               rank orders the point's class: per axis, whether the
 *               footprint reaches the next block and which halves of the two
 *               blocks it covers, ranked so that the points a block receives
 *               from itself and from its -x, -y and -xy neighbours in one
 *               z-chunk are four contiguous key ranges;
 *   bits 23-25 / 26-28  x / y cell of the first tap within its block;
 *   bits 29-31  z cell of the first tap within its 8-cell z-chunk.
 * mn_zsweep_setpts computes the words and fr exactly as mn_setpts_t12 does
 * the cells (crit64, bit for bit); sort them with mn_sort_pairs(key_bits =
 * bits of mn_zsweep_nkeys() - 1, fr as payload) and build zstart
 * (mn_zsweep_nkeys() + 1 int32: zstart[k] = first sorted index with key
 * >= k) with mn_zsweep_starts. The spread reads the sorted words and
 * fractions; strengths are c[perm[j]] (caller order), or c[j] when perm is
 * NULL (c already in sorted order); pre: optional sorted-order multiplier.
 * Products are formed in fp16 hi/lo halves on v_mfma_f32_16x16x32_f16 (three
 * products per term, about 2^-22 relative) and accumulated in f32, with a
 * per-wave power-of-two scale on the strengths, so any finite strength
 * magnitude is handled.
 * ref: nd.py:152-165 (cells), nd.py:492-579 (output-driven spread),
 * nd.py:298-372 (bin sort).
 */
int64_t mn_zsweep_nkeys(const mn_bins *g);
int mn_zsweep_setpts(const mn_bins *g, int64_t P, const double *const x[3], int prec64,
                     uint32_t *word, float *const fr[3], mn_stream_t stream);
int mn_zsweep_starts(const mn_bins *g, int64_t P, const uint32_t *sorted_word, int32_t *zstart,
                     mn_stream_t stream);
int mn_spread_zsweep(const mn_bins *g, float beta, int64_t P, int zseg, const int32_t *zstart,
                     const uint32_t *perm, const uint32_t *sorted_word,
                     const float *const frs[3], const void *c, const void *pre, void *grid,
                     mn_stream_t stream);
/*
 * B strength vectors over one sorted point set: cs holds B rows of P
 * (caller order, or sorted order when perm is NULL), grids B fine grids of
 * n0*n1*n2 complex64, each fully overwritten. One launch covers the vectors
 * in pairs, a wave per (block, pair) sharing the weights and A operands
 * (an odd last vector gets a wave per block of its own). Each grid equals
 * mn_spread_zsweep's for its vector to fp32 rounding (the pair kernel sums
 * the same products in other K-steps; bit for bit with the environment
 * variable MN_ZSWEEP_PAIRS=0, which gives every vector its own wave).
 * ref: nd.py:683-742 (batched output-driven spread), nd.py:744-794.
 */
int mn_spread_zsweep_batch(const mn_bins *g, float beta, int64_t P, int64_t B, int zseg,
                           const int32_t *zstart, const uint32_t *perm,
                           const uint32_t *sorted_word, const float *const frs[3],
                           const void *cs, void *grids, mn_stream_t stream);

/*
 * Z-gather interpolation, the fast path for 3D type-2 on z-sweep geometries
 * (same checks as mn_spread_zsweep). Point state: mn_zgather_setpts writes
 * the z-sweep word with the key ((bx*(n1/8) + by)*ceil(n2/8) + z/8)*16 +
 * 2*(x cell of the first tap in its block) -- the points of a block and
 * z-chunk ordered by that x cell; bits 23-31 as for the spread -- and the
 * fractions; sort and build zstart exactly as for the spread
 * (mn_zsweep_nkeys, mn_sort_pairs, mn_zsweep_starts). Each
 * wavefront owns an 8x8 column block over a z-segment of zseg cells (a
 * positive multiple of 8), holds the (8 + w - 1)^2 window columns x 16
 * z-slots of the grid as fp16 hi/lo MFMA operands (v_mfma_f32_16x16x32_f16,
 * three products per term, about 2^-22 relative, f32 accumulation, a
 * power-of-two scale per 8 z-slots so any finite grid magnitude is handled)
 * and interpolates every point whose first tap lies in the block exactly
 * once; a tile of 16 points runs the matrix cores only over the x columns
 * its footprints cover. grids: B fine grids of n0*n1*n2 complex64; outs: B
 * rows of P complex64, written in caller order (outs[b][perm[j]]).
 * ref: nd.py:974-1073 (output-driven gather), nd.py:298-372 (bin sort).
 */
int mn_zgather_setpts(const mn_bins *g, int64_t P, const double *const x[3], int prec64,
                      uint32_t *word, float *const fr[3], mn_stream_t stream);
int mn_interp_zgather(const mn_bins *g, float beta, int64_t P, int64_t B, int zseg,
                      const int32_t *zstart, const uint32_t *perm, const uint32_t *sorted_word,
                      const float *const frs[3], const void *grids, void *outs,
                      mn_stream_t stream);

/*
 * Owner-computes 2D spread ("y-sweep"), the fast path for 2D type-1 grids
 * with n0 a multiple of 64 (>= 128), w <= 8 and (n0/64)*n1*2 <= 2^26 keys.
 * Each wavefront owns 64 consecutive x-columns over a y-segment of yseg
 * cells, walks y with a w-cell window per column in registers and stores
 * every grid cell once (no atomics; the grids are fully overwritten).
 * B strength vectors (c: B x P, caller order; grid: B x n0 x n1) run in
 * groups of up to 8 per wavefront, which share the point loads, ES weights
 * and batch lists; every vector's result is bit-identical to a B = 1 launch.
 * g: dim 2, w, n (m and nb are not used).
 *
 * Point word (one uint32 per point, from mn_ysweep_setpts):
 *   bits 0-25  key = (bx*n1 + y)*2 + reach, where bx is the 64-column block
 *              of the first tap, y its cell, and reach whether the
 *              footprint crosses into the next block;
 *   bits 26-31 x cell of the first tap within its block.
 * mn_ysweep_setpts computes the words and fr exactly as mn_setpts_t12 does
 * the cells; sort them with mn_sort_pairs (key_bits = bits of
 * mn_ysweep_nkeys() - 1, fr as payload) and build ystart
 * (mn_ysweep_nkeys() + 1 int32) with mn_ysweep_starts. Strengths are
 * c[perm[j]], or c[j] when perm is NULL.
 * ref: nd.py:152-165 (cells), nd.py:492-579 and nd.py:683-742 (output-driven
 * and batched spread), nd.py:298-372 (bin sort).
 */
int64_t mn_ysweep_nkeys(const mn_bins *g);
int mn_ysweep_setpts(const mn_bins *g, int64_t P, const double *const x[2], int prec64,
                     uint32_t *word, float *const fr[2], mn_stream_t stream);
int mn_ysweep_starts(const mn_bins *g, int64_t P, const uint32_t *sorted_word, int32_t *ystart,
                     mn_stream_t stream);
int mn_spread_ysweep(const mn_bins *g, float beta, int64_t P, int64_t B, int yseg,
                     const int32_t *ystart, const uint32_t *perm, const uint32_t *sorted_word,
                     const float *const frs[2], const void *c, void *grid, mn_stream_t stream);

/*
 * 2D owner-computes spread on the matrix cores ("y-window MFMA sweep"):
 * grids[b] (n0 x n1 complex64, fully overwritten) = spread of strength
 * vector b for B vectors (c: B rows of P). For 2D geometries with
 * 2 <= w <= 8, n0 a multiple of 16 (>= 32) and n1 a multiple of 8 (>= 16).
 * One wavefront owns 16 consecutive x-columns over a y-segment of yseg
 * cells (a multiple of 8) and keeps each vector's 16 x 16-slot y-window in
 * matrix-core accumulators: A = the x-weights, B = the strength times the
 * y-weights, both split into fp16 hi + lo (three products, f32
 * accumulation).
 * Point word (one uint32 per point, from mn_ymfma_setpts):
 *   bits 0-24  key = ((x/16)*(n1/8) + y/8)*2 + reach   (sorted on)
 *   bits 25-28 x mod 16 of the first tap; bits 29-31 y mod 8
 * (reach = the footprint crosses into the next 16-column block).
 * mn_ymfma_setpts computes the words and fr exactly as mn_setpts_t12 does
 * i1 and fr; sort the words with mn_sort_pairs (key_bits = bit length of
 * mn_ymfma_nkeys() - 1, fr as payload) and build ystart
 * (mn_ymfma_nkeys() + 1 int32) with mn_ymfma_starts. Strengths are
 * c[perm[j]], or c[j] when perm is NULL; c holds B rows of P values, or P
 * rows of B values when point_major is nonzero (then a point's strengths
 * are one contiguous run, the faster layout for B > 1).
 * ref: nd.py:152-165 (cells), nd.py:492-579 and nd.py:683-742 (output-driven
 * and batched spread), nd.py:298-372 (bin sort).
 */
int64_t mn_ymfma_nkeys(const mn_bins *g);
int mn_ymfma_setpts(const mn_bins *g, int64_t P, const double *const x[2], int prec64,
                    uint32_t *word, float *const fr[2], mn_stream_t stream);
int mn_ymfma_starts(const mn_bins *g, int64_t P, const uint32_t *sorted_word, int32_t *ystart,
                    mn_stream_t stream);
int mn_spread_ymfma(const mn_bins *g, float beta, int64_t P, int64_t B, int yseg,
                    const int32_t *ystart, const uint32_t *perm, const uint32_t *sorted_word,
                    const float *const frs[2], const void *c, int point_major, void *grid,
                    mn_stream_t stream);

/*
 * out (P x B, point-major) = the transpose of in (B x P, vector-major), for
 * B complex64 strength vectors of P points: the layout mn_spread_ymfma
 * reads with point_major = 1, so that a point visit gathers its B
 * strengths as one run. in and out must not overlap.
 * ref: nd.py:683-742 (the reference's batched spread takes the (n_trans, M)
 * strength matrix whole).
 */
int mn_pointmajor_c64(int64_t B, int64_t P, const void *in, void *out, mn_stream_t stream);

/*
 * out[j] = in[perm[j]] for P complex64 values (a strength vector into
 * sorted order). ref: nd.py:603 (mx.take of c by perm, GM spread).
 */
int mn_permute_c64(int64_t P, const uint32_t *perm, const void *in, void *out,
                   mn_stream_t stream);

/*
 * Start index of every bin in the sorted order: starts[b] = first sorted
 * position whose bin key is >= b, for b in [0, nbins] (nbins + 1 int32).
 * ref: nd.py:347-372 (_od_finish bin ranges).
 */
int mn_bin_starts(const mn_bins *g, int64_t P, const uint32_t *sorted_key, int32_t *starts,
                  mn_stream_t stream);

/*
 * Streaming 3D interpolation: as mn_interp, for 3D grids with bins of
 * m = (16, 16, 8) and 2 <= w <= 12. One workgroup owns a 16 x 16 column
 * block and walks its z-bins in order with a sliding LDS window of the grid
 * (the block's columns plus the kernel halo, 8 + w - 1 z-cells deep); each
 * grid cell is read (16 + w - 1)^2 / 256 times. Points sorted by bin key
 * with bin_start from mn_bin_starts; out[perm[j]] receives point j (times
 * post[j] when post is not NULL).
 * ref: nd.py:974-1073 (OD gather), gpu_t3.py:653-693 (type-3 gather x post).
 */
int mn_interp_zstream(const mn_bins *g, float beta, int64_t P, const int32_t *bin_start,
                      const uint32_t *perm, const int32_t *const i1s[3],
                      const float *const frs[3], const void *grid, const void *post, void *out,
                      mn_stream_t stream);

/*
 * Direct 3D interpolation for point sets that are sparse on their grid: one
 * thread per sorted point reads its w^3 taps straight from the complex64
 * grid (w contiguous z-cells per row), with no staged tile. Same inputs and
 * outputs as mn_interp without the subproblem table: points in any order
 * (bin-sorted for locality), out[perm[j]] = interp(point j) (times post[j]
 * when post is not NULL). Only g->dim, g->w and g->n are used.
 * ref: gpu_t3.py:653-693 (t3gather: the type-3 per-target gather x post),
 * nd.py:908-972 (GM gather).
 */
int mn_interp_direct(const mn_bins *g, float beta, int64_t P, const uint32_t *perm,
                     const int32_t *const i1s[3], const float *const frs[3], const void *grid,
                     const void *post, void *out, mn_stream_t stream);

/*
 * Batched spread: B strength vectors cs (B x P, caller order, row-major)
 * over the same points into B grids (B x prod n, overwritten); the ES
 * weights are computed once per point and applied to every vector.
 * ref: nd.py:683-742 (_get_batch_spread), nd.py:744-794 (execute_batch).
 */
int mn_spread_batch(const mn_bins *g, float beta, int64_t P, int64_t nsub,
                    const int32_t *sub_info, const uint32_t *perm,
                    const int32_t *const i1s[3], const float *const frs[3],
                    int64_t B, const void *cs, void *grids, mn_stream_t stream);

/*
 * Interpolation (type-2 core): out[perm[j]] = post[j] * sum over the w^dim
 * taps of grid[cell] * prod_d psi(cell_d - x_j,d); post may be NULL (= 1).
 * One workgroup per subproblem loads its padded tile into LDS once.
 * ref: nd.py:974-1073 + nd.py:1093-1102 (OD gather), nd.py:908-972 (GM
 * gather), gpu_t3.py:653-693 + gpu_t3.py:1337-1343 (type-3 gather x post).
 */
int mn_interp(const mn_bins *g, float beta, int64_t P, int64_t nsub,
              const int32_t *sub_info, const uint32_t *perm,
              const int32_t *const i1s[3], const float *const frs[3],
              const void *grid, const void *post, void *out, mn_stream_t stream);

/*
 * Mode shuffle + deconvolution, type 1: for a batch of grids (n_up) and
 * mode boxes (N, modeord=0, k_d in [-(N_d/2), N_d - N_d/2)):
 * fk[b][m] = grid[b][(m - N/2) mod n_up] * prod_d dec_d[m_d].
 * ref: nd.py:416-435 (t1crop), nd.py:615-621.
 */
int mn_crop_deconv(int dim, const int64_t n_up[3], const int64_t N[3],
                   int64_t batch, const void *grid, const float *const dec[3],
                   void *fk, mn_stream_t stream);

/*
 * Inverse of the above (type 2, and the type-3 inner pad with N = nf):
 * grid[b][r] = fk[b][m] * prod_d dec_d[m_d] where r = (m - N/2) mod n_up,
 * and 0 at every off-band cell. grid is fully overwritten.
 * ref: nd.py:878-906 (t2pad), nd.py:1084-1089, gpu_t3.py:630-651 (t3pad).
 */
int mn_pad_deconv(int dim, const int64_t n_up[3], const int64_t N[3],
                  int64_t batch, const void *fk, const float *const dec[3],
                  void *grid, mn_stream_t stream);

/*
 * Type-3 source setup on the nf grid g (dim 3): per dim
 * xi = ((x - C)/gam)/hd + nf/2 (fp64, numpy operation order), i1, fr,
 * bin key, and the prephase pre[j] = exp(i*isign*(D0 x0 + D1 x1 + D2 x2))
 * (caller order, complex64). prec_flags: bit 0 = coordinate rescale in fp64
 * (else fp32), bit 1 = phase angles in fp64 (else fp32); "crit64" = 3.
 * ref: gpu_t3.py:474-488 (host), gpu_t3.py:237-276 + 508-555 (df64 GPU),
 * gpu_t3.py:345-346 (precision modes).
 */
int mn_t3_setpts_src(const mn_bins *g, int64_t P, const double *const x[3],
                     const double C[3], const double gam[3], const double hd[3],
                     const double D[3], int isign, int prec_flags,
                     int32_t *const i1[3], float *const fr[3], uint32_t *key,
                     void *pre, mn_stream_t stream);

/*
 * Type-3 target setup on the n_up grid g (dim 3, kernel width g->w = w2):
 * theta = (s - D)*hg, lam = theta/h2 + n_up/2, i1, fr, bin key, and
 * post[k] = exp(i*isign*sum_d C_d (s_d - D_d)) / prod_d phihat(theta_d),
 * phihat(xi) = 2 sum_q fq[q] cos(xi dq[q]) with quad = [dq(nquad), fq(nquad)]
 * (device fp64; fq = GL weight * psi(dq) of the outer kernel). prec_flags
 * as for mn_t3_setpts_src.
 * ref: gpu_t3.py:357-377, sizing.py:74-85 (kernel_ft).
 */
int mn_t3_setpts_trg(const mn_bins *g, int64_t M, const double *const s[3],
                     const double D[3], const double hg[3], const double h2[3],
                     const double C[3], int isign, int prec_flags,
                     const double *quad, int nquad, int32_t *const i1[3],
                     float *const fr[3], uint32_t *key, void *post,
                     mn_stream_t stream);

/*
 * e^{i*isign*phi}, phi = sum of ncomp (1..8) fp64 component arrays of n
 * elements (comps is a host array of device pointers), summed and reduced
 * in native fp64 on the GPU; out is complex64.
 * ref: dfmath.py:29-54 (expi_df64 kernel), dfmath.py:57-134 (expi).
 */
int mn_expi(int ncomp, const double *const *comps, int64_t n, int isign,
            void *out, mn_stream_t stream);

/*
 * In-place complex64 FFT of `batch` contiguous C-ordered grids of shape
 * n[0..dim-1]; isign > 0 runs the unnormalised backward transform
 * (e^{+i}), isign < 0 the forward one (e^{-i}). rocFFT plans (and their
 * work buffers) are cached per (device, dim, n, batch, direction).
 * ref: gpu_t3.py:94-148 (fft_axis), nd.py:374-383 (_fft_grid),
 * vkfft_bridge/vkfft_bridge.cpp:25-71 (plan cache + in-place execute).
 */
int mn_fft_exec(int dim, const int64_t n[3], int64_t batch, int isign,
                void *data, mn_stream_t stream);

/*
 * Pruned, deconvolving FFTs for power-of-two fine grids (16 <= n[d] <= 4096;
 * mn_fftp_supported). One pass per axis transforms that axis's lines and
 * keeps (type 1) or fills (type 2) only the N[d] modes of modeord 0
 * (k = i - N[d]/2 at FFT index k mod n[d]), multiplied by dec[d][i]:
 *   mn_fft_crop_deconv: fk = crop(FFT(grid)) * dec0 x dec1 x dec2; grid is
 *     read only (batch grids of prod n -> batch mode boxes of prod N);
 *   mn_pad_deconv_fft:  grid = FFT(pad(fk * dec0 x dec1 x dec2)).
 * isign > 0 is the unnormalised e^{+i} transform, isign < 0 e^{-i}. work
 * (device) holds the intermediate arrays: mn_fftp_work_bytes(...) bytes,
 * 8*batch*(n0*n1*N2 + n0*N1*N2) in 3D. Replaces FFT + crop (or pad + FFT):
 * at n = 2N a 3D type-1 pass set moves 2.8 GB instead of 8.9 GB.
 * ref: nd.py:374-383 (_fft_grid), nd.py:416-435 (crop/deconv kernel),
 * nd.py:878-906 (pad/deconv), gpu_t3.py:94-148 (fft_axis).
 */
int mn_fftp_supported(int dim, const int64_t n[3]);
int64_t mn_fftp_work_bytes(int dim, const int64_t n[3], const int64_t N[3], int64_t batch);
int mn_fft_crop_deconv(int dim, const int64_t n_up[3], const int64_t N[3], int64_t batch,
                       int isign, const void *grid, const float *const dec[3], void *work,
                       int64_t work_bytes, void *fk, mn_stream_t stream);
int mn_pad_deconv_fft(int dim, const int64_t n_up[3], const int64_t N[3], int64_t batch,
                      int isign, const void *fk, const float *const dec[3], void *work,
                      int64_t work_bytes, void *grid, mn_stream_t stream);
/*
 * The same transform in double precision (complex128 data, rocFFT double).
 * The type-3 pipeline runs its inner-grid FFT this way: its target
 * deconvolution 1/phihat(theta) reaches ~1e2 at the band edges and
 * amplifies an fp32 FFT's absolute roundoff there (cfg-5-like workloads:
 * 7.5e-5 relative error in fp32 against 1.6e-5 in fp64).
 * ref: gpu_t3.py:94-148 (the type-3 FFT stage).
 */
int mn_fft_exec_f64(int dim, const int64_t n[3], int64_t batch, int isign, void *data,
                    mn_stream_t stream);

/*
 * pad/deconv in double precision: grid = pad(fk * dec0 x dec1 x dec2) with
 * fk and grid complex128 and fp64 factors, ahead of mn_fft_exec_f64; and
 * out = (complex64) in for n complex128 values, after it.
 * ref: gpu_t3.py:630-651 (type-3 inner-grid pad + deconvolution).
 */
int mn_pad_deconv_c128(int dim, const int64_t n_up[3], const int64_t N[3], int64_t batch,
                       const void *fk, const double *const dec[3], void *grid,
                       mn_stream_t stream);
int mn_round_c64(int64_t n, const void *in, void *out, mn_stream_t stream);

/*
 * Batched zero-padding line FFTs in double precision: one axis pass of the
 * type-3 inner-grid transform, with that axis's pad and deconvolution fused.
 * `in` is complex128 of shape (A, nin, B), C order; `out` has shape
 * (A, n, B) when out_layout == 0, (n, A*B) with the line index fastest when
 * out_layout == 1, or (A*B, n) with each line's n values contiguous when
 * out_layout == 2; complex128, or complex64 when out_c64 != 0. Line (a, b) is
 * in[a, :, b]: element m, times dec[m] (fp64, length nin; NULL for none),
 * sits at FFT index (m - nin/2) mod n with zeros elsewhere, and
 *   out[a, r, b] = sum_p x[p] exp(isign 2 pi i p r / n)   (unnormalised).
 * Three passes (z, y, x) of bf (nf0 nf1 nf2) give
 * FFT(pad(bf * dec0 x dec1 x dec2)) on n_up without a padded fp64 grid
 * (the x pass in layout 2 writes it as (n1, n2, n0), x innermost, in whole
 * lines instead of runs of B's low power of two).
 * n must be 2^a 3^b 5^c in [2, 8192] (mn_fft64_lines_supported), 1 <= nin <=
 * n, A*B < 2^31, and in and out must not overlap. The twiddle tables are
 * cached per (device, n, sign) and released by mn_fft_cache_clear.
 * ref: gpu_t3.py:630-651 (t3pad), gpu_t3.py:94-148 (fft_axis),
 * gpu_t3.py:697-741 (t3padz: the slab path's fused pad, deconvolution and
 * z-DFT).
 */
int mn_fft64_lines_supported(int64_t n);
int mn_fft64_lines(int64_t A, int64_t nin, int64_t B, int64_t n, int isign, const void *in,
                   const double *dec, void *out, int out_c64, int out_layout,
                   mn_stream_t stream);

/*
 * Batched transpose of complex128 matrices: out[b][c][r] = in[b][r][c] for
 * in (Bt, R, C) and out (Bt, C, R), Bt <= 65535; in and out must not
 * overlap. Between the type-3 line passes it turns a strided axis of long
 * lines (which fill the LDS one line per workgroup) into a contiguous one.
 * ref: gpu_t3.py:151-199 (fft_axis_scrambled: the reference's four-step
 * reordering for long axes).
 */
int mn_transpose_c128(int64_t Bt, int64_t R, int64_t C, const void *in, void *out,
                      mn_stream_t stream);

/* Destroy all cached FFT plans and line-FFT twiddle tables (call with no
 * transform in flight). */
int mn_fft_cache_clear(void);

/* Zero `bytes` bytes of device memory with a fill kernel (no memset node). */
int mn_fill_zero(void *ptr, int64_t bytes, mn_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MLX_NUFFT_AMD_H */
