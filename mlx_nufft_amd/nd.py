"""Type-1/2 NUFFT plans in 1, 2 and 3 dims on the MI355X engine.

    type 1:  f[k] = sum_j c[j] exp(i*isign * k . x_j)
    type 2:  c[j] = sum_k f[k] exp(i*isign * k . x_j)

with k_d in [-(N_d//2), (N_d-1)//2] (modeord=0, even or odd N_d) and any x
(folded mod 2pi in fp64). Mirrors the reference's Type1PlanND/Type2PlanND
(ref: mlx_nufft/nd.py:94-1119): the constructor is setpts, execute runs
the transform; all device work is HIP kernels behind the C-ABI.

Pipeline (type 1): fp64 setpts (fold, rescale, cell/frac, sort key) ->
stable radix sort carrying the point data -> ES spread (3D: owner-computes
z-sweep, no atomics; otherwise LDS tiles flushed with atomics) -> FFT with
the mode crop and deconvolution fused (pruned per-axis FFT on power-of-two
grids, else rocFFT + crop). Type 2 runs the adjoint chain: deconvolve +
zero-pad + FFT -> LDS-tiled interpolation written straight to caller order.
"""

import os

import numpy as np
import torch

from . import _engine as E
from . import _lib as L
from .sizing import kernel_ft, kernel_params, next235even

PI = np.pi


def _as_coord_tuple(x):
    if isinstance(x, (np.ndarray, torch.Tensor)) and x.ndim == 1:
        x = (x,)
    return tuple(x)


class PlanArgumentError(ValueError, AssertionError):
    """An invalid plan option. It is a ValueError; it is an AssertionError as
    well because the reference rejects these options with assert
    statements (ref: nd.py:399, 871; types12.py:36-37), so callers that
    catch either keep working."""


SPREAD_METHODS = ("auto", "od", "gm")


def od_applicable(dim, w, n_up, P):
    """The reference's rule for when its output-driven (bin-tiled) spread and
    interp apply: w <= 8, at least 20000 points, and a padded bin tile of
    m + w cells per dim (m = 2048 in 1D, 48 - w in 2D, 15 - w in 3D) that
    fits 28 KB and the fine grid (ref: nd.py:281-305, 329). A forced
    spread_method="od" outside it raises ValueError, as there; the engine's
    own kernels apply more widely."""
    if w > 8 or P < 20000:
        return False
    m = {1: [2048], 2: [48 - w] * 2, 3: [15 - w] * 3}[dim]
    tile = [mi + w for mi in m]
    return (min(m) >= 1 and 8 * int(np.prod(tile)) <= 28 * 1024
            and all(n >= t for n, t in zip(n_up, tile)))


class _PointsND:
    """Shared point/kernel setup for ND types 1 and 2 (ref: nd.py:94-150)."""

    def __init__(self, x, n_modes, eps, isign, upsampfac, prec, sort_points):
        if prec not in ("fp32", "crit64"):
            raise PlanArgumentError("prec must be 'fp32' or 'crit64'")
        x = _as_coord_tuple(x)
        self.dim = len(x)
        if self.dim not in (1, 2, 3):
            raise ValueError("dims 1, 2, 3 supported")
        if np.isscalar(n_modes):
            n_modes = (int(n_modes),) * self.dim
        self.N = tuple(int(n) for n in n_modes)
        if len(self.N) != self.dim:
            raise ValueError(f"n_modes length {len(self.N)} must match dim {self.dim}")
        if any(n < 1 for n in self.N):
            raise ValueError("mode dims must be >= 1")
        if upsampfac in (None, 0, 0.0):
            upsampfac = 2.0
        if not 1.0 < upsampfac <= 4.0:
            raise ValueError(f"upsampfac must be in (1, 4], got {upsampfac}")
        self.prec = prec
        self.isign = +1 if isign >= 0 else -1
        self.eps = eps
        self.sigma = upsampfac
        self.w, self.beta = kernel_params(eps, upsampfac)
        self.n_up = [next235even(max(2 * self.w, int(np.ceil(upsampfac * n)))) for n in self.N]
        self._sort_points = bool(sort_points)
        self.profile = False
        self.profile_deferred = False
        self.last_profile = {}
        self._deferred = []

        npts = x[0].numel() if isinstance(x[0], torch.Tensor) else np.size(x[0])
        if self.spread_method == "od" and not od_applicable(self.dim, self.w, self.n_up, npts):
            raise ValueError(f"spread_method='od' does not apply here (w={self.w}, "
                             f"n_up={tuple(self.n_up)}, P={npts}): it needs w <= 8, "
                             f"P >= 20000 and a fine grid at least one padded bin wide")

        self.device = L.require_gpu()
        x64 = self._coords(x)
        self.P = x64[0].numel()
        self._stream_interp = self._use_zstream and E.zstream_eligible(self.dim, self.w)
        if self._stream_interp:
            self.bins = E.make_bins(3, self.w, self.n_up, m=E.ZSTREAM_M)
        else:
            self.bins = E.make_bins(self.dim, self.w, self.n_up, cell_bytes=self._cell_bytes)
        self._zsweep = E.zsweep_eligible(self.dim, self.w, self.n_up) and self._zsweep_wanted()
        if self._zsweep:
            self._zbins = E.make_bins(3, self.w, self.n_up, m=(8, 8, 1))
        # 2D: the y-window MFMA sweep where its geometry applies, else the
        # VALU y-sweep
        self._ymfma = self._use_zsweep and E.ymfma_eligible(self.dim, self.w, self.n_up)
        self._ysweep = self._use_zsweep and (self._ymfma or
                                             E.ysweep_eligible(self.dim, self.w, self.n_up))
        if self._ysweep:
            self._ybins = E.make_bins(2, self.w, self.n_up, m=(16 if self._ymfma else 64, 1))
        self._set_points(x64)

        # Mode deconvolution 1/phihat(2 pi k / n_up) on the uncentred fine grid
        # (points folded into [0, 2pi), so no (-1)^k factor). rocFFT's backward
        # transform is unnormalised, so no prod(n_up) factor is folded in
        # (ref: nd.py:136-149 folds it because its ifft divides by n).
        self.decs = []
        for d in range(self.dim):
            k = np.arange(-(self.N[d] // 2), self.N[d] - self.N[d] // 2, dtype=np.float64)
            self.decs.append(1.0 / kernel_ft(2.0 * PI * k / self.n_up[d], self.beta, self.w))
        self.dev_dec = [torch.from_numpy(v.astype(np.float32)).to(self.device) for v in self.decs]
        self._grid = None
        self._pruned = E.fftp_supported(self.n_up)
        self._work = None

    # the z-sweep point state is built in the spread's key order unless set
    _zgather_points = False

    def _zsweep_wanted(self):
        """Whether the point state should be the z-sweep's (3D, eligible grids)."""
        return self._use_zsweep

    # -- point state -------------------------------------------------------

    def _coords(self, x):
        x64 = [L.to_dev_f64(v, self.device) for v in x]
        P = x64[0].numel()
        if P < 1:
            raise ValueError("at least one nonuniform point is required")
        if not all(v.numel() == P for v in x64):
            raise ValueError("coordinate arrays must have equal length")
        return x64

    def _compute_cells_gpu(self, x64):
        """Unsorted device (i1 int32, fr fp32) lists per dim for fp64 coords,
        bit-exact with the reference's host fp64 path (ref: nd.py:152-165)."""
        if not isinstance(x64[0], torch.Tensor):
            x64 = [L.to_dev_f64(v, self.device) for v in x64]
        i1, fr, _ = E.setpts_t12(self.bins, x64, self.prec == "crit64")
        return [i1[d] for d in range(self.dim)], [fr[d] for d in range(self.dim)]

    def _compute_cells(self, x64):
        """numpy mirrors self.i1 / self.fr of the cell setup (caller order)."""
        i1, fr = self._compute_cells_gpu(x64)
        self.i1 = [v.cpu().numpy() for v in i1]
        self.fr = [v.cpu().numpy() for v in fr]

    def _set_points(self, x64):
        tm = self._timer()
        if self._zsweep:
            with tm("setpts+sort+tables"):
                prev = getattr(self, "pts", None)
                gather = self._zgather_points
                kind = "zgather" if gather else "zsweep"
                same = isinstance(prev, E.ZSweepPoints) and prev.kind == kind
                self.pts = E.ZSweepPoints(self._zbins, x64, self.prec == "crit64",
                                          prev=prev if same else None, gather=gather)
                del prev
        elif self._ysweep:
            with tm("setpts+sort+tables"):
                prev = getattr(self, "pts", None)
                self.pts = E.YSweepPoints(self._ybins, x64, self.prec == "crit64",
                                          prev=prev if isinstance(prev, E.YSweepPoints) else None,
                                          mfma=self._ymfma)
                del prev
        else:
            with tm("setpts"):
                i1, fr, key = E.setpts_t12(self.bins, x64, self.prec == "crit64")
            with tm("sort+tables"):
                self.pts = E.SortedPoints(self.bins, i1, fr, key, stream=self._stream_interp)
                del i1, fr, key
        self.sorted = True
        self._od = True
        self._finish_profile(tm, "setpts")
        self.last_setpts_profile = dict(self.last_profile) if self.profile else {}

    @property
    def mx_perm(self):
        """Device permutation (sorted position -> caller index)."""
        return self.pts.perm

    @property
    def perm(self):
        return self.pts.perm.cpu().numpy().astype(np.intp)

    def _fine_grid(self, batch=1):
        shape = (batch, *self.n_up)
        if self._grid is None or tuple(self._grid.shape) != shape:
            self._grid = None
            self._grid = torch.empty(shape, dtype=torch.complex64, device=self.device)
        return self._grid

    def _fft_work(self, batch=1):
        """Work buffer of the pruned FFT (intermediate per-axis arrays)."""
        nbytes = E.fftp_work_bytes(self.n_up, self.N, batch)
        if nbytes <= 0:
            return None
        if self._work is None or self._work.numel() < nbytes:
            self._work = None
            self._work = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        return self._work

    def _timer(self):
        return E.StageTimer(self.profile)

    def _finish_profile(self, tm, kind="execute"):
        """With profile on, per-stage HIP-event times of the last call land in
        last_profile (one stream synchronisation). With profile_deferred as
        well, the events are kept unread (no synchronisation) until
        drain_profiles()."""
        if not self.profile:
            return
        if self.profile_deferred:
            self._deferred.append((kind, tm))
            self.last_profile = {}
        else:
            self.last_profile = tm.times_ms()

    def drain_profiles(self):
        """[(kind, {stage: ms})] of the deferred calls, in call order (one
        synchronisation); kind is "setpts" or "execute"."""
        torch.cuda.synchronize()
        out = [(kind, tm.times_ms(sync=False)) for kind, tm in self._deferred]
        self._deferred = []
        return out


class Type1PlanND(_PointsND):
    """f[k] = sum_j c[j] exp(i*isign * k . x_j), modeord=0 box, dims 1-3.

    ref: nd.py:386-855.
    """

    _cell_bytes = E.SPREAD_CELL_BYTES
    _use_zstream = False

    def __init__(self, x, n_modes, eps=1e-6, isign=+1, upsampfac=2.0, prec="crit64",
                 sort_points=True, spread_method="auto"):
        """spread_method: "auto" picks the fastest spread for the geometry
        (3D: the owner-computes z-sweep; 2D: the y-sweep; else LDS tiles);
        "od" does the same but first raises ValueError where the reference's
        output-driven spread would not apply; "gm" forces the LDS-tile
        spread with its atomic flush, this engine's counterpart of the
        reference's global-memory atomic spread (ref: nd.py:397-404)."""
        if spread_method not in SPREAD_METHODS:
            raise PlanArgumentError(f"spread_method must be one of {SPREAD_METHODS}, got "
                                    f"{spread_method!r}")
        self.spread_method = spread_method
        self._use_zsweep = spread_method != "gm"
        super().__init__(x, n_modes, eps, isign, upsampfac, prec, sort_points)

    def _strengths(self, c):
        cd = L.to_dev_c64(c, self.device).reshape(-1)
        if cd.numel() != self.P:
            raise ValueError(f"c.size ({cd.numel()}) must equal the number of nonuniform "
                             f"points ({self.P})")
        return cd

    def execute(self, c, return_np=True):
        """ref: nd.py:581-625."""
        cd = self._strengths(c)
        grid = self._fine_grid(1)
        fk = torch.empty(self.N, dtype=torch.complex64, device=self.device)
        tm = self._timer()
        self._spread_one(self.pts, cd, grid, tm)
        self._fft_crop(grid, fk, tm, 1)
        self._finish_profile(tm)
        return L.to_host(fk) if return_np else fk

    def _spread_one(self, pts, cd, grid, tm):
        """grid = spread of cd (caller order) over the points of pts."""
        if pts.kind == "zsweep":
            with tm("spread"):
                E.spread_zsweep(pts, self.beta, cd, grid)
        elif pts.kind == "ysweep":
            with tm("spread"):
                E.spread_ysweep(pts, self.beta, cd, grid)
        elif pts.kind == "ymfma":
            with tm("spread"):
                E.spread_ymfma(pts, self.beta, cd, grid)
        else:
            with tm("zero"):
                E.fill_zero(grid)
            with tm("spread"):
                E.spread(pts, self.beta, cd, grid, accumulate=True)

    def _fft_crop(self, grid, fk, tm, batch):
        if self._pruned:
            with tm("fft"):
                E.fft_crop_deconv(self.n_up, self.N, grid, self.dev_dec, fk, self.isign,
                                  self._fft_work(batch), batch=batch)
            return
        with tm("fft"):
            E.fft(grid, self.n_up, self.isign, batch=batch)
        with tm("deconv"):
            E.crop_deconv(self.n_up, self.N, grid, self.dev_dec, fk, batch=batch)

    def execute_batch(self, cs, return_np=True):
        """B strength vectors over the same points: one shared spread (ES
        weights once per point), one batched FFT, one batched crop.
        cs: (B, P) -> (B, *N). ref: nd.py:744-794."""
        if isinstance(cs, torch.Tensor):
            shape = tuple(cs.shape)
        else:
            cs = np.asarray(cs)
            shape = cs.shape
        if len(shape) != 2 or shape[1] != self.P:
            raise ValueError(f"cs must have shape (B, {self.P})")
        B = int(shape[0])
        cd = L.to_dev_c64(cs, self.device).reshape(B, self.P)
        grids = self._fine_grid(B)
        fk = torch.empty((B, *self.N), dtype=torch.complex64, device=self.device)
        tm = self._timer()
        with tm("spread"):
            if self.pts.kind == "zsweep":
                E.spread_zsweep_batch(self.pts, self.beta, cd, grids)
            elif self.pts.kind == "ysweep":
                E.spread_ysweep(self.pts, self.beta, cd, grids)
            elif self.pts.kind == "ymfma":
                E.spread_ymfma(self.pts, self.beta, cd, grids)
            else:
                E.spread_batch(self.pts, self.beta, cd, grids)
        self._fft_crop(grids, fk, tm, B)
        self._finish_profile(tm)
        return L.to_host(fk) if return_np else fk

    def set_sources(self, x, backend="host"):
        """Re-point the plan to new coordinates, keeping kernels, deconvolution
        and FFT plans; P may change. Both backends run the same bit-exact
        native-fp64 device setup (the reference's "host" is its fp64 numpy
        path, "gpu" its df64 Metal path). Returns self. ref: nd.py:627-681."""
        x = _as_coord_tuple(x)
        if len(x) != self.dim:
            raise ValueError(f"expected {self.dim} coordinate arrays, got {len(x)}")
        if backend not in ("host", "gpu"):
            raise ValueError(f"unknown backend {backend!r}")
        x64 = [L.to_dev_f64(v, self.device) for v in x]
        P = x64[0].numel()
        if P < 1 or not all(v.numel() == P for v in x64):
            raise ValueError("coordinate arrays must be non-empty, equal length")
        self.P = P
        if not (isinstance(self.pts, (E.ZSweepPoints, E.YSweepPoints)) and self.pts.P == P):
            self.pts = None  # nothing to reuse: free the old point state first
        self._set_points(x64)
        return self

    def execute_disjoint(self, c, groups, return_np=True):
        """G independent transforms of disjoint point subsets of one plan:
        out[g] = type-1 of c restricted to {j : groups[j] == g}, G =
        max(groups) + 1, (G, *N); points with a negative label belong to no
        subset and empty subsets give zeros. Every point is spread once in
        total: the plan's sorted point state is partitioned by label with
        one stable sort, each subset keeps the spread's key order, and the
        subsets are spread one after another into one fine grid, each
        followed by its own FFT and crop (ref: nd.py:796-855)."""
        if isinstance(groups, torch.Tensor):
            gl = groups.to(device=self.device, dtype=torch.int64)
        else:
            gl = torch.from_numpy(np.asarray(groups).astype(np.int64)).to(self.device)
        if tuple(gl.shape) != (self.P,):
            raise ValueError(f"groups must have shape ({self.P},)")
        cd = self._strengths(c)
        G = int(gl.max()) + 1 if gl.numel() else 0
        out = torch.zeros((max(G, 0), *self.N), dtype=torch.complex64, device=self.device)
        if G > 0:
            split = E.GroupSplit(self.pts, gl, G)
            del gl
            grid = self._fine_grid(1)
            tm = self._timer()
            for g, sub in split:
                self._spread_one(sub, cd, grid, tm)
                self._fft_crop(grid, out[g], tm, 1)
            self._finish_profile(tm)
        return L.to_host(out) if return_np else out


class Type2PlanND(_PointsND):
    """c[j] = sum_k f[k] exp(i*isign * k . x_j), modeord=0 box, dims 1-3.

    ref: nd.py:858-1119.
    """

    _cell_bytes = E.INTERP_CELL_BYTES
    _use_zsweep = False
    _use_zstream = True
    _zgather_points = True

    def __init__(self, x, n_modes, eps=1e-6, isign=-1, upsampfac=2.0, prec="crit64",
                 sort_points=False, spread_method="auto"):
        """spread_method selects the interpolation: "auto" the staged-tile
        gather (or, for 3D points sparse on their grid, the direct gather);
        "od" the same after raising ValueError where the reference's
        output-driven gather would not apply; "gm" the direct gather, which
        reads each point's taps straight from the grid as the reference's
        global-memory gather does (3D; 1D and 2D keep the tiles)
        (ref: nd.py:869-874). sort_points is accepted for the interface: the
        gathers always run in bin order and write results in caller order,
        which is the order the reference returns for either value."""
        if spread_method not in SPREAD_METHODS:
            raise PlanArgumentError(f"spread_method must be one of {SPREAD_METHODS}, got "
                                    f"{spread_method!r}")
        self.spread_method = spread_method
        super().__init__(x, n_modes, eps, isign, upsampfac, prec, sort_points)

    def execute(self, fk, return_np=True):
        """ref: nd.py:1075-1119."""
        fd = L.to_dev_c64(fk, self.device).reshape(-1)
        ntot = int(np.prod(self.N))
        if fd.numel() != ntot:
            raise ValueError(f"f.size ({fd.numel()}) must equal the mode-box size "
                             f"{tuple(self.N)}")
        grid = self._fine_grid(1)
        out = torch.empty(self.P, dtype=torch.complex64, device=self.device)
        tm = self._timer()
        if self._pruned:
            with tm("fft"):
                E.pad_deconv_fft(self.n_up, self.N, fd, self.dev_dec, grid, self.isign,
                                 self._fft_work(1))
        else:
            with tm("deconv"):
                E.pad_deconv(self.n_up, self.N, fd, self.dev_dec, grid)
            with tm("fft"):
                E.fft(grid, self.n_up, self.isign)
        with tm("interp"):
            if self.pts.kind == "zgather":
                E.interp_zgather(self.pts, self.beta, grid, out)
            elif self._gather_direct():
                E.interp_direct(self.pts, self.beta, grid, out)
            else:
                E.interp(self.pts, self.beta, grid, out)
        self._finish_profile(tm)
        return L.to_host(out) if return_np else out

    def _zsweep_wanted(self):
        """The z-gather interpolation (over the z-sweep point state) serves
        "auto" and "od" plans whose points are dense enough on their grid
        (E.zgather_preferred); MN_INTERP=tiles or zstream keeps those gathers."""
        if self.dim != 3 or self.spread_method not in ("auto", "od"):
            return False
        if os.environ.get("MN_INTERP", "") in ("tiles", "zstream"):
            return False
        return E.zgather_preferred(self.P, self.w, self.n_up)

    def _gather_direct(self):
        """3D points sparse on the fine grid read their taps directly (no
        staged tiles); decided once per point set."""
        pts = self.pts
        if getattr(self, "_gd_pts", None) is not pts:
            self._gd_pts = pts
            if pts.kind == "zgather":
                self._gd = False
            elif self.spread_method == "gm":
                self._gd = self.dim == 3
            else:
                self._gd = E.interp_direct_preferred(pts, self.w, self.n_up)
        return self._gd
