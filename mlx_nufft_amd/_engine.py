"""Thin wrappers over the C-ABI used by the plan classes: point setup, the
stable bin sort, subproblem tables, spread/interp, deconvolution, FFT and
expi. Every function takes and returns torch device tensors and runs on the
current stream; shapes are validated by the C side as well.

Bin geometry (the tile a workgroup owns) is chosen here, per dim and kernel
width, from the LDS budget of one CDNA4 workgroup.
"""

import contextlib
import ctypes
import os

import numpy as np
import torch

from . import _lib as L

_require = L.require

MSUB = 1024                 # max points per spread/interp subproblem
TILE_BUDGET = 80 * 1024     # LDS bytes for one padded tile (2 workgroups/CU)


_budget = None


def tile_budget():
    """LDS bytes for one tile: TILE_BUDGET, capped by the device limit."""
    global _budget
    if _budget is None:
        try:
            dev = int(L.lib().mn_device_lds_bytes())
        except RuntimeError:
            dev = TILE_BUDGET
        _budget = min(TILE_BUDGET, dev if dev > 0 else 65536)
    return _budget


SPREAD_CELL_BYTES = 16   # spread tiles accumulate complex values in fp64
INTERP_CELL_BYTES = 8    # interp tiles hold complex64 grid values


def bin_sizes(dim, w, n_up, cell_bytes=SPREAD_CELL_BYTES, npts=None):
    """Bin size m per dim: the padded tile (m + w - 1 cells per dim,
    cell_bytes each) must fit tile_budget() bytes of LDS. npts (the number
    of points, when known) lets the 3D interp tiles grow for sparse points.
    Overridable with the environment variable MN_BIN_M="m0,m1,m2" (tuning)."""
    budget = tile_budget()
    env = os.environ.get("MN_BIN_M")
    if env:
        m = [int(v) for v in env.split(",")]
        m = (m + [m[-1]] * 3)[:dim]
    elif dim == 1:
        m = [1024]
    elif dim == 2:
        m = [32, 32]
    elif cell_bytes == INTERP_CELL_BYTES:
        # interp is bound by staging tiles: small bins keep about 9
        # workgroups resident per CU, which beats the smaller halo re-read of
        # big tiles (MI355X, 3D type 2 at 512^3: 2.0 ms at m = 8, 3.1 ms at
        # 16). Along z (the contiguous axis) the padded tile row is made 17
        # cells for w >= 5: rows of 16 (and 12) cells put the lane pairs'
        # LDS reads on conflicting banks. Type-2 execute, 2e7 points on
        # 512^3, m = (8, 8, m2): w = 5: 2.11 ms at m2 = 8, 1.94 at 13;
        # w = 6: 2.44 at 8, 2.35 at 12, 3.07 at 11; w = 7: 3.13 at 8, 3.03
        # at 11, 4.19 at 10. At w = 4, 8 is best within 2 %.
        # Sparse points (under 0.1 per cell, as type-3 targets) leave few
        # points per bin, so the tile load dominates and wider bins re-read
        # less halo: cfg 5's targets (1e6 on 240^3, w = 9) gather in 0.276 ms
        # with m = (11, 11, 9), 0.289 with 10^3, 0.318 with 9^3, 0.361 with
        # (8, 8, 9).
        mxy = 11 if (dim == 3 and npts is not None
                     and npts < 0.1 * float(np.prod([float(n) for n in n_up]))) else 8
        m = [mxy, mxy, max(8, 18 - w) if w >= 5 else 8]
    else:
        side = int(round((budget / cell_bytes) ** (1.0 / 3.0) - 1e-9))
        while cell_bytes * side ** 3 > budget:
            side -= 1
        m = [max(1, side - w + 1)] * 3
    m = [max(1, min(int(mi), int(n))) for mi, n in zip(m, n_up)]
    while cell_bytes * int(np.prod([mi + w - 1 for mi in m])) > budget and max(m) > 1:
        k = int(np.argmax(m))
        m[k] -= 1
    return m


def make_bins(dim, w, n_up, m=None, cell_bytes=SPREAD_CELL_BYTES, npts=None):
    if m is None:
        m = bin_sizes(dim, w, n_up, cell_bytes, npts=npts)
    return L.Bins.make(dim, w, list(n_up), m)


def key_bits(bins):
    return max(1, int(bins.nbins - 1).bit_length())


def _rows(t, dim):
    return [t[d] for d in range(dim)]


def setpts_t12(bins, xs, prec64):
    """Cells, fractions and bin keys of type-1/2 points (caller order)."""
    dim, P = bins.dim, xs[0].numel()
    dev = xs[0].device
    i1 = torch.empty((dim, P), dtype=torch.int32, device=dev)
    fr = torch.empty((dim, P), dtype=torch.float32, device=dev)
    key = torch.empty(P, dtype=torch.int32, device=dev)
    L.check(L.lib().mn_setpts_t12(ctypes.byref(bins), P, L.ptr3(xs), int(bool(prec64)),
                                  L.ptr3(_rows(i1, dim)), L.ptr3(_rows(fr, dim)), L.ptr(key),
                                  L.stream()), "setpts")
    return i1, fr, key


def sort_keys(key, nbits):
    """Stable argsort of uint32 keys (stored in int32 tensors): (sorted, perm)."""
    skey, perm, _ = sort_pairs(key, nbits, [])
    return skey, perm


def sort_pairs(key, nbits, cols, outs=None, skey=None, perm=None, ws=None):
    """Stable sort of uint32 keys on their low nbits bits, carrying 32-bit
    payload columns (int32/float32 tensors of P elements) into outs:
    (sorted keys, perm, sorted columns). Outputs and the workspace are new
    tensors unless given."""
    P = key.numel()
    lib = L.lib()
    ncols = len(cols)
    ws_bytes = int(lib.mn_sort_pairs_workspace_bytes(P, ncols))
    if ws is None or ws.numel() < ws_bytes:
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=key.device)
    skey = torch.empty_like(key) if skey is None else skey
    perm = torch.empty_like(key) if perm is None else perm
    if outs is None:
        outs = [torch.empty_like(c) for c in cols]
    cin = (ctypes.c_void_p * max(1, ncols))(*[c.data_ptr() for c in cols])
    cout = (ctypes.c_void_p * max(1, ncols))(*[c.data_ptr() for c in outs])
    L.check(lib.mn_sort_pairs(P, int(nbits), L.ptr(key), L.ptr(skey), L.ptr(perm), ncols, cin,
                              cout, L.ptr(ws), ws.numel(), L.stream()), "sort")
    return skey, perm, outs


def gather_points(perm, i1, fr, extra=None):
    dim, P = i1.shape
    i1s = torch.empty_like(i1)
    frs = torch.empty_like(fr)
    ext = torch.empty_like(extra) if extra is not None else None
    L.check(L.lib().mn_gather_points(dim, P, L.ptr(perm), L.ptr3(_rows(i1, dim)),
                                     L.ptr3(_rows(fr, dim)), L.ptr3(_rows(i1s, dim)),
                                     L.ptr3(_rows(frs, dim)), L.ptr(extra), L.ptr(ext),
                                     L.stream()), "gather_points")
    return i1s, frs, ext


def build_subproblems(bins, skey, msub=MSUB):
    """(info[nsub, 3] = (bin, start, count), nsub). Blocks on one 8-byte read."""
    P = skey.numel()
    lib = L.lib()
    max_sub = bins.nbins + P // msub + 1
    info = torch.empty((max_sub, 3), dtype=torch.int32, device=skey.device)
    ws = torch.empty(int(lib.mn_subproblem_workspace_bytes(ctypes.byref(bins))),
                     dtype=torch.uint8, device=skey.device)
    nsub = ctypes.c_int64(0)
    L.check(lib.mn_build_subproblems(ctypes.byref(bins), P, L.ptr(skey), int(msub), L.ptr(info),
                                     max_sub, ctypes.byref(nsub), L.ptr(ws), ws.numel(),
                                     L.stream()), "subproblems")
    return info, int(nsub.value)


ZSTREAM_M = (16, 16, 8)  # bins of the streaming 3D interpolation


def zstream_eligible(dim, w):
    """True when the streaming 3D interpolation is selected (MN_INTERP=zstream,
    3D, 2 <= w <= 12). It reads the grid 1.7x instead of 4.3x, but measured
    slower than 8^3 tiles at 2e7 points / 512^3 (2.2 vs 2.0 ms: its window
    slides are not cache-line aligned and random gathers conflict in LDS),
    so the tiles are the default."""
    if os.environ.get("MN_INTERP", "") != "zstream":
        return False
    return dim == 3 and 2 <= w <= 12


class SortedPoints:
    """Bin-sorted point state of one point set on one fine grid: sorted cells
    and fractions, perm, and either the subproblem table (tiles) or the
    start of every bin (kind "zstream", bins of ZSTREAM_M)."""

    def __init__(self, bins, i1, fr, key, extra=None, msub=MSUB, stream=False):
        self.kind = "zstream" if stream else "tiles"
        self.bins = bins
        self.P = i1.shape[1]
        dim = bins.dim
        self.i1s = torch.empty_like(i1)
        self.frs = torch.empty_like(fr)
        cols = _rows(i1, dim) + _rows(fr, dim)
        outs = _rows(self.i1s, dim) + _rows(self.frs, dim)
        if extra is not None:
            cols += [extra.real.contiguous(), extra.imag.contiguous()]
            outs += [torch.empty_like(cols[-2]), torch.empty_like(cols[-1])]
        skey, self.perm, out = sort_pairs(key, key_bits(bins), cols, outs)
        self.extra = torch.complex(out[2 * dim], out[2 * dim + 1]) if extra is not None else None
        del out, outs, cols
        if stream:
            self.bstart = torch.empty(bins.nbins + 1, dtype=torch.int32, device=key.device)
            L.check(L.lib().mn_bin_starts(ctypes.byref(bins), self.P, L.ptr(skey),
                                          L.ptr(self.bstart), L.stream()), "bin starts")
            self.info, self.nsub = None, 0
        else:
            self.bstart = None
            self.info, self.nsub = build_subproblems(bins, skey, msub)
        self.skey = skey

    def i1_rows(self):
        return _rows(self.i1s, self.bins.dim)

    def fr_rows(self):
        return _rows(self.frs, self.bins.dim)


def fill_zero(t):
    L.check(L.lib().mn_fill_zero(L.ptr(t), t.numel() * t.element_size(), L.stream()),
            "fill_zero")


# z-segment (cells) owned by one z-sweep wavefront: each segment also sweeps
# the chunk below it, and 256 halves that overhead against 128 (measured on
# MI355X at 512^3: 1.48 -> 1.40 ms, 512 no better)
ZSEG = 256


def zsweep_eligible(dim, w, n_up):
    """True when the owner-computes z-sweep spread applies: 3D, w <= 8, the
    x and y fine-grid sizes multiples of 8 (>= 16) and at most 2^23 sort keys
    ((n0/8)(n1/8) ceil(n2/8) 16, e.g. 512^3 or 1024^2 x 256). MN_SPREAD=tiles
    forces the LDS-tile spread instead."""
    if os.environ.get("MN_SPREAD", "") == "tiles":
        return False
    if dim != 3 or w > 8 or not all(n % 8 == 0 and n >= 16 for n in n_up[:2]) or n_up[2] < 8:
        return False
    return (n_up[0] // 8) * (n_up[1] // 8) * (-(-n_up[2] // 8)) * 16 <= 1 << 23


class ZSweepPoints:
    """Point state for the z-sweep spread (gather=False, kind "zsweep") or
    the z-gather interpolation (gather=True, kind "zgather"): packed point
    words and fractions (setpts), stably sorted together by the z-sweep key
    (points of a block and z-chunk grouped by class for the spread, ordered
    by the x cell of their first tap for the gather), and the key start
    table. Given the previous point set of the same plan (prev) with the
    same P and geometry, its device buffers are reused, so re-pointing
    allocates nothing; prev's contents are overwritten in stream order."""

    def __init__(self, bins, x64, prec64, prev=None, gather=False):
        lib = L.lib()
        dev = x64[0].device
        self.kind = "zgather" if gather else "zsweep"
        self.bins = bins
        self.P = P = x64[0].numel()
        self.K = K = int(lib.mn_zsweep_nkeys(ctypes.byref(bins)))
        same = (prev is not None and prev.P == P and prev.K == K and prev.dev == dev)
        self.dev = dev
        self._bufs = bufs = prev._bufs if same else {}

        def buf(name, shape, dtype):
            if name not in bufs:
                bufs[name] = torch.empty(shape, dtype=dtype, device=dev)
            return bufs[name]

        word = buf("word_in", P, torch.int32)
        fr = buf("fr_in", (3, P), torch.float32)
        setpts = lib.mn_zgather_setpts if gather else lib.mn_zsweep_setpts
        L.check(setpts(ctypes.byref(bins), P, L.ptr3(x64), int(bool(prec64)), L.ptr(word),
                       L.ptr3(_rows(fr, 3)), L.stream()), f"{self.kind} setpts")
        self.frs = buf("frs", (3, P), torch.float32)
        ws_bytes = int(lib.mn_sort_pairs_workspace_bytes(P, 3))
        self.word, self.perm, _ = sort_pairs(
            word, max(1, (K - 1).bit_length()), _rows(fr, 3), _rows(self.frs, 3),
            skey=buf("word", P, torch.int32), perm=buf("perm", P, torch.int32),
            ws=buf("ws", ws_bytes, torch.uint8))
        self.zstart = buf("zstart", K + 1, torch.int32)
        L.check(lib.mn_zsweep_starts(ctypes.byref(bins), P, L.ptr(self.word), L.ptr(self.zstart),
                                     L.stream()), "zsweep starts")

    def fr_rows(self):
        return _rows(self.frs, 3)


def ysweep_eligible(dim, w, n_up):
    """True when the owner-computes y-sweep spread applies: 2D, w <= 8, the x
    fine-grid size a multiple of 64 (>= 128) and at most 2^26 sort keys
    ((n0/64)*n1*2). MN_SPREAD=tiles forces the LDS-tile spread instead."""
    if os.environ.get("MN_SPREAD", "") == "tiles":
        return False
    return (dim == 2 and 2 <= w <= 8 and n_up[0] % 64 == 0 and n_up[0] >= 128
            and n_up[1] >= w and (n_up[0] // 64) * n_up[1] * 2 <= 1 << 26)


def ymfma_eligible(dim, w, n_up):
    """True when the 2D spread on the matrix cores (y-window MFMA sweep)
    applies: 2D, w <= 8, n0 a multiple of 16 (>= 32), n1 a multiple of 8
    (>= 16) and at most 2^25 sort keys ((n0/16)*(n1/8)*2). MN_SPREAD=tiles
    forces the LDS-tile spread, MN_SPREAD=ysweep the VALU y-sweep."""
    if os.environ.get("MN_SPREAD", "") in ("tiles", "ysweep"):
        return False
    return (dim == 2 and 2 <= w <= 8 and n_up[0] % 16 == 0 and n_up[0] >= 32
            and n_up[1] % 8 == 0 and 16 <= n_up[1] < 1 << 24
            and (n_up[0] // 16) * (n_up[1] // 8) * 2 <= 1 << 25)


class YSweepPoints:
    """Point state for the 2D y-sweep spread (mfma=False, kind "ysweep") or
    the y-window MFMA sweep (mfma=True, kind "ymfma"): packed point words and
    fractions, stably sorted together by the sweep's key, and the key start
    table. Buffers of the previous point set of the same plan (prev, same
    kind, P and geometry) are reused, as in ZSweepPoints."""

    def __init__(self, bins, x64, prec64, prev=None, mfma=False):
        lib = L.lib()
        dev = x64[0].device
        self.kind = "ymfma" if mfma else "ysweep"
        nkeys, setpts, starts = ((lib.mn_ymfma_nkeys, lib.mn_ymfma_setpts, lib.mn_ymfma_starts)
                                 if mfma else
                                 (lib.mn_ysweep_nkeys, lib.mn_ysweep_setpts, lib.mn_ysweep_starts))
        self.bins = bins
        self.P = P = x64[0].numel()
        self.K = K = int(nkeys(ctypes.byref(bins)))
        same = (prev is not None and prev.kind == self.kind and prev.P == P and prev.K == K
                and prev.dev == dev)
        self.dev = dev
        self._bufs = bufs = prev._bufs if same else {}

        def buf(name, shape, dtype):
            if name not in bufs:
                bufs[name] = torch.empty(shape, dtype=dtype, device=dev)
            return bufs[name]

        V2 = ctypes.c_void_p * 2
        word = buf("word_in", P, torch.int32)
        fr = buf("fr_in", (2, P), torch.float32)
        L.check(setpts(ctypes.byref(bins), P, V2(x64[0].data_ptr(), x64[1].data_ptr()),
                       int(bool(prec64)), L.ptr(word), V2(fr[0].data_ptr(), fr[1].data_ptr()),
                       L.stream()), f"{self.kind} setpts")
        self.frs = buf("frs", (2, P), torch.float32)
        ws_bytes = int(lib.mn_sort_pairs_workspace_bytes(P, 2))
        self.word, self.perm, _ = sort_pairs(
            word, max(1, (K - 1).bit_length()), _rows(fr, 2), _rows(self.frs, 2),
            skey=buf("word", P, torch.int32), perm=buf("perm", P, torch.int32),
            ws=buf("ws", ws_bytes, torch.uint8))
        self.ystart = buf("ystart", K + 1, torch.int32)
        L.check(starts(ctypes.byref(bins), P, L.ptr(self.word), L.ptr(self.ystart), L.stream()),
                f"{self.kind} starts")

    def fr_rows(self):
        return _rows(self.frs, 2)


class _Subset:
    """Points [s, e) of a group-sorted copy of a point state: the attributes
    the spread entry points read, as views of the copy's columns (frs and
    i1s are lists of per-dimension rows)."""

    def __init__(self, kind, bins, P, **views):
        self.kind = kind
        self.bins = bins
        self.P = P
        self.__dict__.update(views)

    def fr_rows(self):
        return list(self.frs)

    def i1_rows(self):
        return list(self.i1s)


class GroupSplit:
    """A point state partitioned by group label, for spreads of disjoint
    point subsets that visit every point once in total.

    glabel: int64 labels in caller order; labels outside [0, G) are left
    out. One stable sort by label (carrying the spread's sorted columns)
    keeps each group's points in the state's key order, so each group is a
    contiguous, still key-sorted range. Iterating yields (g, subset) for the
    non-empty groups and builds the subset's start table just before it is
    used: z-/y-sweep key starts in one shared buffer (rebuilt in stream
    order, after the previous group's spread has read it), or the tile
    spread's subproblem table."""

    def __init__(self, pts, glabel, G):
        self.pts = pts
        self.G = G
        dim = pts.bins.dim
        gs = glabel[pts.perm.long()]
        gkey = torch.where((gs < 0) | (gs >= G), G, gs).to(torch.int32)
        del gs
        if pts.kind in ("zsweep", "ysweep", "ymfma"):
            cols = [pts.word, pts.perm] + _rows(pts.frs, dim)
        elif pts.kind == "tiles":
            cols = [pts.skey, pts.perm] + _rows(pts.frs, dim) + _rows(pts.i1s, dim)
        else:
            raise ValueError(f"no disjoint spread for point state {pts.kind!r}")
        skey, _, self.cols = sort_pairs(gkey, max(1, int(G).bit_length()), cols)
        del gkey
        bounds = torch.arange(G + 1, dtype=torch.int32, device=skey.device)
        self.starts = torch.searchsorted(skey, bounds).cpu().tolist()
        self._startbuf = None

    def __iter__(self):
        pts, dim, lib, c = self.pts, self.pts.bins.dim, L.lib(), self.cols
        for g in range(self.G):
            s, e = self.starts[g], self.starts[g + 1]
            if e == s:
                continue
            frs = [r[s:e] for r in c[2:2 + dim]]
            if pts.kind == "tiles":
                sub = _Subset("tiles", pts.bins, e - s, perm=c[1][s:e], skey=c[0][s:e], frs=frs,
                              i1s=[r[s:e] for r in c[2 + dim:2 + 2 * dim]])
                sub.info, sub.nsub = build_subproblems(pts.bins, sub.skey)
                yield g, sub
                continue
            if self._startbuf is None:
                self._startbuf = torch.empty(pts.K + 1, dtype=torch.int32,
                                             device=pts.perm.device)
            sub = _Subset(pts.kind, pts.bins, e - s, perm=c[1][s:e], word=c[0][s:e], frs=frs,
                          K=pts.K)
            starts_fn = {"zsweep": lib.mn_zsweep_starts, "ysweep": lib.mn_ysweep_starts,
                         "ymfma": lib.mn_ymfma_starts}[pts.kind]
            L.check(starts_fn(ctypes.byref(pts.bins), sub.P, L.ptr(sub.word),
                              L.ptr(self._startbuf), L.stream()), f"{pts.kind} starts")
            if pts.kind == "zsweep":
                sub.zstart = self._startbuf
            else:
                sub.ystart = self._startbuf
            yield g, sub


def ysweep_vectors_per_wave(B):
    """Vectors one y-sweep wavefront carries (the kernel's rule): the
    largest of 8, 4, 2, 1 not above B."""
    return 8 if B >= 8 else 4 if B >= 4 else 2 if B >= 2 else 1


def ysweep_segment(n_up, B):
    """y-segment per wavefront: the longest power of two (<= 256) that still
    gives at least 8192 / VB wavefronts (VB vectors per wavefront), but at
    least 32 (each segment re-reads the w - 1 rows below it to warm its
    window). Measured at 2048^2, 1e7 points, w = 7: 32 for B = 1 (0.49 ms;
    0.58 at 16, 0.84 at 64); 64 for B = 8, VB = 8 (2.19 ms; 2.39 at 32)."""
    vb = ysweep_vectors_per_wave(B)
    groups = -(-B // vb)
    nbx = n_up[0] // 64
    yseg = 256
    while yseg > 32 and nbx * (-(-n_up[1] // yseg)) * groups * vb < 8192:
        yseg //= 2
    return yseg


def spread_ysweep(pts, beta, cs, grids):
    """grids[b] = spread(cs[b]) for B vectors (cs: (B, P) or (P,), caller
    order) with the 2D y-sweep; grids are fully overwritten."""
    B = 1 if cs.dim() == 1 else int(cs.shape[0])
    n_up = [int(pts.bins.n[0]), int(pts.bins.n[1])]
    V2 = ctypes.c_void_p * 2
    L.check(L.lib().mn_spread_ysweep(ctypes.byref(pts.bins), float(beta), pts.P, B,
                                     ysweep_segment(n_up, B), L.ptr(pts.ystart), L.ptr(pts.perm),
                                     L.ptr(pts.word), V2(pts.frs[0].data_ptr(), pts.frs[1].data_ptr()),
                                     L.ptr(cs), L.ptr(grids), L.stream()), "spread_ysweep")


def ymfma_segment(n_up, B):
    """y-segment per wavefront of the y-window MFMA sweep: the longest power
    of two (<= 256, >= 32) that still gives at least 4096 wavefronts (each
    segment also sweeps the chunk below it)."""
    vb = ysweep_vectors_per_wave(B)
    groups = -(-B // vb)
    nbx = n_up[0] // 16
    yseg = 256
    while yseg > 32 and nbx * (-(-n_up[1] // yseg)) * groups < 4096:
        yseg //= 2
    return yseg


def spread_ymfma(pts, beta, cs, grids):
    """grids[b] = spread(cs[b]) for B vectors (cs: (B, P) or (P,), caller
    order) with the y-window MFMA sweep; grids are fully overwritten. Several
    vectors are first transposed to point-major (P, B), so that a point
    visit gathers its strengths in one run rather than one sector per
    vector."""
    B = 1 if cs.dim() == 1 else int(cs.shape[0])
    n_up = [int(pts.bins.n[0]), int(pts.bins.n[1])]
    V2 = ctypes.c_void_p * 2
    pm = 0
    if B > 1:
        _require(cs.is_contiguous() and cs.dtype == torch.complex64,
                 "spread_ymfma: cs must be a contiguous complex64 (B, P) tensor")
        ct = torch.empty((int(cs.shape[1]), B), dtype=torch.complex64, device=cs.device)
        L.check(L.lib().mn_pointmajor_c64(B, int(cs.shape[1]), L.ptr(cs), L.ptr(ct), L.stream()),
                "pointmajor")
        cs = ct
        pm = 1
    L.check(L.lib().mn_spread_ymfma(ctypes.byref(pts.bins), float(beta), pts.P, B,
                                    ymfma_segment(n_up, B), L.ptr(pts.ystart), L.ptr(pts.perm),
                                    L.ptr(pts.word), V2(pts.frs[0].data_ptr(), pts.frs[1].data_ptr()),
                                    L.ptr(cs), pm, L.ptr(grids), L.stream()), "spread_ymfma")


def permute_c64(perm, c, out):
    """out[j] = c[perm[j]] (complex64 strengths into sorted order)."""
    L.check(L.lib().mn_permute_c64(perm.numel(), L.ptr(perm), L.ptr(c), L.ptr(out), L.stream()),
            "permute")


def spread_zsweep(pts, beta, c, grid, pre=None, zseg=ZSEG, presorted=False):
    """grid = spread(c) with the owner-computes z-sweep (overwrites grid).
    c is in caller order, or in sorted order when presorted."""
    L.check(L.lib().mn_spread_zsweep(ctypes.byref(pts.bins), float(beta), pts.P, int(zseg),
                                     L.ptr(pts.zstart), None if presorted else L.ptr(pts.perm),
                                     L.ptr(pts.word), L.ptr3(pts.fr_rows()), L.ptr(c), L.ptr(pre),
                                     L.ptr(grid), L.stream()), "spread_zsweep")


def spread_zsweep_batch(pts, beta, cs, grids, zseg=ZSEG, presorted=False):
    """grids[b] = spread(cs[b]) for B vectors with the z-sweep, one launch
    with a wave per (block, vector) (overwrites grids)."""
    B = cs.shape[0]
    _require(grids.shape[0] == B and cs.shape[1] == pts.P and cs.is_contiguous()
             and grids.is_contiguous(), "spread_zsweep_batch: cs must be (B, P) and grids "
             "(B, n0, n1, n2), both contiguous")
    L.check(L.lib().mn_spread_zsweep_batch(ctypes.byref(pts.bins), float(beta), pts.P, B,
                                           int(zseg), L.ptr(pts.zstart),
                                           None if presorted else L.ptr(pts.perm),
                                           L.ptr(pts.word), L.ptr3(pts.fr_rows()), L.ptr(cs),
                                           L.ptr(grids), L.stream()), "spread_zsweep_batch")


def spread(pts, beta, c, grid, pre=None, accumulate=False):
    """grid = spread(c) (or grid += spread(c) with accumulate=True)."""
    fn = L.lib().mn_spread_accumulate if accumulate else L.lib().mn_spread
    L.check(fn(ctypes.byref(pts.bins), float(beta), pts.P, pts.nsub, L.ptr(pts.info),
               L.ptr(pts.perm), L.ptr3(pts.i1_rows()), L.ptr3(pts.fr_rows()), L.ptr(c),
               L.ptr(pre), L.ptr(grid), L.stream()), "spread")


def spread_c128(pts, beta, c, grid128, pre=None):
    """grid128 (complex128) = spread(c) with fp64 products and accumulation."""
    L.check(L.lib().mn_spread_c128(ctypes.byref(pts.bins), float(beta), pts.P, pts.nsub,
                                   L.ptr(pts.info), L.ptr(pts.perm), L.ptr3(pts.i1_rows()),
                                   L.ptr3(pts.fr_rows()), L.ptr(c), L.ptr(pre), L.ptr(grid128),
                                   L.stream()), "spread_c128")


def t3_tile_bins(w, n):
    """Bins of the type-3 LDS-tile spread. With w <= 16 the matrix-core
    kernel takes the tiles, so bins are 17 - w cells wide: padded tiles of 16
    cells per dim (one 16 x 16 MFMA tile per x plane). MN_T3_TILE_MFMA=0
    selects the LDS-atomic kernel and the LDS budget's bins instead."""
    if w <= 16 and os.environ.get("MN_T3_TILE_MFMA", "") != "0":
        return make_bins(3, w, n, m=[max(1, min(17 - w, int(k))) for k in n])
    return make_bins(3, w, n, cell_bytes=SPREAD_CELL_BYTES)


OWNER_M = 16   # owner-computes spread bins: 16^3 fp64 complex cells = 64 KB of LDS


def owner_bins(w, n):
    """Owner-computes spread bins: 16 cells per dim, except a last dim of at
    most 18 cells, which stays whole (one bin along it: no split columns and
    no second z-owner per point; 16*16*18 cells still fit two workgroups per
    CU)."""
    m = [min(OWNER_M, k) for k in n]
    if n[2] <= 18:
        m[2] = n[2]
    return make_bins(3, w, n, m=m)


def spread_owner_c128(pts, beta, c, grid128, pre=None):
    """Owner-computes 3D spread into a complex128 grid that it fully
    overwrites (no zero fill); pts must carry bin starts (kind "zstream")."""
    _require(pts.bstart is not None and grid128.dtype == torch.complex128
             and grid128.numel() >= int(np.prod([pts.bins.n[d] for d in range(3)])),
             "spread_owner_c128: needs a point state with bin starts and a complex128 grid of "
             "the fine-grid size")
    L.check(L.lib().mn_spread_owner_c128(ctypes.byref(pts.bins), float(beta), pts.P,
                                         L.ptr(pts.bstart), L.ptr(pts.perm), L.ptr3(pts.i1_rows()),
                                         L.ptr3(pts.fr_rows()), L.ptr(c),
                                         None if pre is None else L.ptr(pre), L.ptr(grid128),
                                         L.stream()), "spread_owner_c128")


def spread_batch(pts, beta, cs, grids):
    L.check(L.lib().mn_spread_batch(ctypes.byref(pts.bins), float(beta), pts.P, pts.nsub,
                                    L.ptr(pts.info), L.ptr(pts.perm), L.ptr3(pts.i1_rows()),
                                    L.ptr3(pts.fr_rows()), int(cs.shape[0]), L.ptr(cs),
                                    L.ptr(grids), L.stream()), "spread_batch")


def interp_direct(pts, beta, grid, out, post=None):
    """3D gather without staged tiles: one thread per sorted point reads its
    w^3 taps from the grid (sparse point sets)."""
    L.check(L.lib().mn_interp_direct(ctypes.byref(pts.bins), float(beta), pts.P, L.ptr(pts.perm),
                                     L.ptr3(pts.i1_rows()), L.ptr3(pts.fr_rows()), L.ptr(grid),
                                     L.ptr(post), L.ptr(out), L.stream()), "interp direct")


def interp_direct_preferred(pts, w, n_up):
    """True when the direct gather should beat the staged one: its w^3 taps
    per point against the staged path's padded tile per subproblem (or ~1.7
    reads of the grid for the z-streaming path). Measured on MI355X (taps /
    staged cells: staged ms, direct ms): 11.4: 0.43, 0.53 (1e6 targets on
    240^3); 2.3-2.6: 2.62, 2.20 and 6.43, 3.14 (4e6 targets on 640^3 and on
    5400^2 x 24); 0.6: 2.42, 0.74 and 4.17, 1.19 (1e6 targets on the same
    grids). The crossover lies between 2.6 and 11.4; 5 is used."""
    if pts.bins.dim != 3:
        return False
    direct = float(pts.P) * w ** 3
    if pts.kind == "zstream":
        staged = 1.7 * float(np.prod([float(n) for n in n_up]))
    else:
        staged = float(pts.nsub) * float(np.prod([pts.bins.m[d] + w - 1 for d in range(3)]))
    return direct < 5.0 * staged


def zgather_preferred(P, w, n_up):
    """True when the z-gather interpolation should beat the direct gather for
    P points on the 3D fine grid n_up: the direct gather reads P w^3 taps,
    the z-gather (8 + w - 1)^2 columns of 8 new z-cells for every 8x8-column
    block and z-chunk that holds points (16 after a skipped chunk), expected
    over uniform points. The factor 5 is the crossover measured between the
    direct and the staged-tile gathers (interp_direct_preferred)."""
    nchunks = (n_up[0] / 8.0) * (n_up[1] / 8.0) * -(-n_up[2] // 8)
    lam = float(P) / nchunks
    busy = nchunks * -np.expm1(-lam)
    staged = (8 + w - 1) ** 2 * 8.0 * busy * (1.0 + np.exp(-lam))
    return float(P) * w ** 3 >= 5.0 * staged


def interp_zgather(pts, beta, grids, outs, B=1, zseg=ZSEG):
    """3D interpolation over the z-sweep point state: B grids (B x n_up)
    into B output vectors of P values in caller order (outs: B x P)."""
    L.check(L.lib().mn_interp_zgather(ctypes.byref(pts.bins), float(beta), pts.P, int(B),
                                      int(zseg), L.ptr(pts.zstart), L.ptr(pts.perm),
                                      L.ptr(pts.word), L.ptr3(pts.fr_rows()), L.ptr(grids),
                                      L.ptr(outs), L.stream()), "interp_zgather")


def interp(pts, beta, grid, out, post=None):
    if pts.kind == "zstream":
        L.check(L.lib().mn_interp_zstream(ctypes.byref(pts.bins), float(beta), pts.P,
                                          L.ptr(pts.bstart), L.ptr(pts.perm),
                                          L.ptr3(pts.i1_rows()), L.ptr3(pts.fr_rows()),
                                          L.ptr(grid), L.ptr(post), L.ptr(out), L.stream()),
                "interp")
        return
    L.check(L.lib().mn_interp(ctypes.byref(pts.bins), float(beta), pts.P, pts.nsub,
                              L.ptr(pts.info), L.ptr(pts.perm), L.ptr3(pts.i1_rows()),
                              L.ptr3(pts.fr_rows()), L.ptr(grid), L.ptr(post), L.ptr(out),
                              L.stream()), "interp")


def crop_deconv(n_up, N, grid, decs, fk, batch=1):
    dim = len(N)
    L.check(L.lib().mn_crop_deconv(dim, L.i64x3(n_up), L.i64x3(N), int(batch), L.ptr(grid),
                                   L.ptr3(decs), L.ptr(fk), L.stream()), "crop_deconv")


def pad_deconv(n_up, N, fk, decs, grid, batch=1):
    dim = len(N)
    L.check(L.lib().mn_pad_deconv(dim, L.i64x3(n_up), L.i64x3(N), int(batch), L.ptr(fk),
                                  L.ptr3(decs), L.ptr(grid), L.stream()), "pad_deconv")


def fftp_supported(n_up):
    """True when the pruned per-axis FFT applies (power-of-two fine grid
    sizes in [16, 4096]); MN_FFT=rocfft forces full rocFFT + crop/pad."""
    if os.environ.get("MN_FFT", "") == "rocfft":
        return False
    return bool(L.lib().mn_fftp_supported(len(n_up), L.i64x3(n_up)))


def fftp_work_bytes(n_up, N, batch=1):
    return int(L.lib().mn_fftp_work_bytes(len(N), L.i64x3(n_up), L.i64x3(N), int(batch)))


def fft_crop_deconv(n_up, N, grid, decs, fk, isign, work, batch=1):
    """fk = crop(FFT(grid)) * prod_d dec_d with the pruned per-axis FFT."""
    L.check(L.lib().mn_fft_crop_deconv(len(N), L.i64x3(n_up), L.i64x3(N), int(batch), int(isign),
                                       L.ptr(grid), L.ptr3(decs), L.ptr(work),
                                       0 if work is None else work.numel(), L.ptr(fk),
                                       L.stream()), "fft_crop_deconv")


def pad_deconv_fft(n_up, N, fk, decs, grid, isign, work, batch=1):
    """grid = FFT(pad(fk * prod_d dec_d)) with the pruned per-axis FFT."""
    L.check(L.lib().mn_pad_deconv_fft(len(N), L.i64x3(n_up), L.i64x3(N), int(batch), int(isign),
                                      L.ptr(fk), L.ptr3(decs), L.ptr(work),
                                      0 if work is None else work.numel(), L.ptr(grid),
                                      L.stream()), "pad_deconv_fft")


def pad_deconv_c128(n_up, N, fk128, decs64, grid128, batch=1):
    """grid128 = pad(fk128 * prod_d dec_d), complex128 with fp64 factors."""
    L.check(L.lib().mn_pad_deconv_c128(len(N), L.i64x3(n_up), L.i64x3(N), int(batch), L.ptr(fk128),
                                       L.ptr3(decs64), L.ptr(grid128), L.stream()),
            "pad_deconv_c128")


def fft_f64(grid128, n_up, isign, batch=1):
    """In-place complex128 FFT (rocFFT double precision)."""
    L.check(L.lib().mn_fft_exec_f64(len(n_up), L.i64x3(n_up), int(batch), int(isign),
                                    L.ptr(grid128), L.stream()), "fft_f64")


def round_c64(src128, out64):
    L.check(L.lib().mn_round_c64(src128.numel(), L.ptr(src128), L.ptr(out64), L.stream()),
            "round_c64")


def fft64_lines_supported(n):
    return bool(L.lib().mn_fft64_lines_supported(int(n)))


FFT64_LAYOUTS = {"anb": 0, "lines_last": 1, "lines_first": 2}


def fft64_lines(A, nin, B, n, isign, src128, dec64, out, layout="anb"):
    """One axis pass of the zero-padding fp64 line FFT: src128 (A, nin, B)
    complex128 -> out (A, n, B) ("anb"), (n, A*B) with the line index fastest
    ("lines_last") or (A*B, n) with each line contiguous ("lines_first"),
    complex128 or complex64 (by out's dtype)."""
    _require(layout in FFT64_LAYOUTS, f"fft64_lines: layout must be one of {tuple(FFT64_LAYOUTS)}")
    c64 = out.dtype == torch.complex64
    _require(src128.dtype == torch.complex128 and src128.numel() >= A * nin * B,
             f"fft64_lines: src must be complex128 with at least {A * nin * B} elements")
    _require(out.numel() >= A * n * B and (c64 or out.dtype == torch.complex128),
             f"fft64_lines: out must be complex64/128 with at least {A * n * B} elements")
    _require(dec64 is None or (dec64.dtype == torch.float64 and dec64.numel() >= nin),
             f"fft64_lines: dec must be float64 with at least {nin} elements")
    L.check(L.lib().mn_fft64_lines(int(A), int(nin), int(B), int(n), int(isign), L.ptr(src128),
                                   None if dec64 is None else L.ptr(dec64), L.ptr(out), int(c64),
                                   FFT64_LAYOUTS[layout], L.stream()), "fft64_lines")


def transpose_c128(Bt, R, C, src, out):
    """out[b][c][r] = src[b][r][c] for complex128 (Bt, R, C) -> (Bt, C, R)."""
    _require(src.dtype == torch.complex128 and out.dtype == torch.complex128,
             "transpose_c128: src and out must be complex128")
    _require(src.numel() >= Bt * R * C and out.numel() >= Bt * R * C,
             f"transpose_c128: src and out need at least {Bt * R * C} elements")
    L.check(L.lib().mn_transpose_c128(int(Bt), int(R), int(C), L.ptr(src), L.ptr(out),
                                      L.stream()), "transpose_c128")


def fft(grid, n_up, isign, batch=1):
    L.check(L.lib().mn_fft_exec(len(n_up), L.i64x3(n_up), int(batch), int(isign), L.ptr(grid),
                                L.stream()), "fft")


def expi(comps, isign, out):
    arr = (ctypes.c_void_p * len(comps))(*[c.data_ptr() for c in comps])
    L.check(L.lib().mn_expi(len(comps), arr, comps[0].numel(), int(isign), L.ptr(out),
                            L.stream()), "expi")


class StageTimer:
    """Optional per-stage HIP-event timing on the current stream."""

    def __init__(self, enabled):
        self.enabled = enabled
        self.events = []

    @contextlib.contextmanager
    def __call__(self, name):
        if not self.enabled:
            yield
            return
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        yield
        b.record()
        self.events.append((name, a, b))

    def times_ms(self, sync=True):
        if sync:
            torch.cuda.synchronize()
        out = {}
        for name, a, b in self.events:
            out[name] = out.get(name, 0.0) + a.elapsed_time(b)
        return out
