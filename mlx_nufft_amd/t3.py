"""Type-3 3D NUFFT plan (nonuniform -> nonuniform) on the MI355X engine.

    f[k] = sum_j c[j] exp(i*isign * s_k . x_j)

FINUFFT-structured like the reference (ref: mlx_nufft/gpu_t3.py:287-1364):
sources are rescaled onto an nf^3 grid, pre-phased by exp(i isign D.x) and
spread; the grid is deconvolved and zero-padded to n_up^3, FFT'd, and
interpolated at the rescaled targets, then multiplied by the post factor
exp(i isign C.(s-D)) / prod_d phihat(theta_d). Plan setup (sizing scalars,
mode deconvolution vectors) is host fp64; per-point setup (source and target
rescale, phases, phihat at every target) is native fp64 on the GPU. The
prephase is fused into the spread and the post factor into the gather.

The deconvolve + pad + FFT stage runs as three fp64 line-FFT passes (z, y,
x) that each transform only the lines that can be non-zero, with that
axis's zero padding and deconvolution fused into the line load and the last
pass rounding to complex64 (csrc/mn_fftl.hip). It never materialises a
padded fp64 grid; this is the role of the reference's slab mode
(gpu_t3.py:697-1041: fused pad, deconv and z-DFT, then per-slab lateral
FFTs), generalised to every axis. Axes longer than 8192 or not 5-smooth
fall back to pad + rocFFT. When an x or y line is long (> 1365 points), the
passes run in reversed axis order with one transpose, so every long line is
read contiguously, and the grid comes out as (n2, n1, n0); otherwise the x
pass stores each x line whole and the grid comes out as (n1, n2, n0). The
targets are set up with their axes in the grid's order. MI355X holds every grid the reference
handles in HBM, so there is no slab switch.
"""

import os
import warnings

import numpy as np
import torch

from . import _engine as E
from . import _lib as L
from .nd import PlanArgumentError
from .sizing import (inner_kernel_params, kernel_ft, kernel_params, next235even,
                     quadrature, set_nhg_type3)

PI = np.pi
_SLAB_THRESHOLD = 3e9   # the reference's slab switch (bytes); informational here
_PREC_FLAGS = {"fp32": 0, "coords64": 1, "phases64": 2, "crit64": 3}


class GpuT3Plan:
    def __init__(self, x, s, eps=1e-5, isign=+1, upsampfac=1.25, prec="crit64",
                 sigma_inner=None, sort_points=True, low_mem=None, source_extent=None,
                 fft_backend="mlx"):
        """x: 3 source coordinate arrays (P,), s: 3 target arrays (M,).

        source_extent: optional [(lo, hi)] * 3 bounds to size the plan for,
        so set_sources() accepts later frames inside them.
        fft_backend: "mlx" (the built-in rocFFT path on this engine) or
        "vkfft" (not available on this platform: raises RuntimeError).
        ref: gpu_t3.py:288-441.
        """
        # the reference asserts these (gpu_t3.py:303-304); PlanArgumentError is
        # both a ValueError and an AssertionError and is not stripped by -O
        if prec not in _PREC_FLAGS:
            raise PlanArgumentError(f"prec must be one of {tuple(_PREC_FLAGS)}, got {prec!r}")
        if fft_backend not in ("mlx", "vkfft"):
            raise PlanArgumentError(f"fft_backend must be 'mlx' or 'vkfft', got {fft_backend!r}")
        if fft_backend == "vkfft":
            raise RuntimeError("the VkFFT-Metal FFT backend is not available on this "
                               "platform; use fft_backend='mlx' (rocFFT)")
        self.fft_backend = fft_backend
        self.prec = prec
        self._flags = _PREC_FLAGS[prec]
        self.isign = int(np.sign(isign))
        self.eps = eps
        self.sigma = upsampfac
        self.w, self.beta = kernel_params(eps, upsampfac)
        if sigma_inner is None or sigma_inner == upsampfac:
            self.sigma_in = upsampfac
            self.w2, self.beta2 = self.w, self.beta
        else:
            self.sigma_in = sigma_inner
            self.w2, self.beta2 = inner_kernel_params(eps, sigma_inner)
        self.device = L.require_gpu()
        self.profile = False
        self.last_profile = {}

        x = tuple(x)
        s = tuple(s)
        if len(x) != 3 or len(s) != 3:
            raise ValueError("type-3 plans take 3 source and 3 target coordinate arrays")
        x64 = [L.to_dev_f64(v, self.device) for v in x]
        s64 = [L.to_dev_f64(v, self.device) for v in s]
        self.P = x64[0].numel()
        self.M = s64[0].numel()
        if self.P < 1 or self.M < 1:
            raise ValueError("type-3 needs at least one source and one target")
        if not all(v.numel() == self.P for v in x64) or not all(v.numel() == self.M for v in s64):
            raise ValueError("coordinate arrays must have equal length")

        # ---- sizing (host fp64 scalars; ref: gpu_t3.py:326-342) -----------
        smin = [float(v.min()) for v in s64]
        smax = [float(v.max()) for v in s64]
        if source_extent is not None:
            self._xext = [(float(lo), float(hi)) for lo, hi in source_extent]
        else:
            self._xext = [(float(v.min()), float(v.max())) for v in x64]
        self.nf, self.gam, self.C, self.D = [], [], [], []
        for d in range(3):
            xlo, xhi = self._xext[d]
            C = 0.5 * (xlo + xhi)
            D = 0.5 * (smin[d] + smax[d])
            X = 0.5 * (xhi - xlo)
            S = 0.5 * (smax[d] - smin[d])
            nf, _, gam = set_nhg_type3(S, X, upsampfac, self.w)
            self.nf.append(nf)
            self.gam.append(gam)
            self.C.append(C)
            self.D.append(D)
        self.n_up = [next235even(int(np.ceil(self.sigma_in * nf))) for nf in self.nf]
        self.slab_mode = False

        # ---- inner-grid transform: three fused pad + deconvolve + line-FFT
        # passes when every axis length is 2^a 3^b 5^c <= 8192 and the line
        # counts fit, else pad + rocFFT (MN_T3_FFT=rocfft forces the latter).
        # When an x or y line is too long for two lines per LDS tile, the
        # passes run in reversed axis order so that every long line is
        # contiguous (z written axis-outermost, y, a transpose, x): the grid
        # then comes out as (n2, n1, n0) and the targets are set up with
        # their axes reversed to gather from it.
        nf, nu = self.nf, self.n_up
        self.fft_lines = (os.environ.get("MN_T3_FFT", "lines") != "rocfft"
                          and all(E.fft64_lines_supported(n) for n in nu)
                          and nf[0] * nf[1] < 2**31 and nf[0] * nu[2] < 2**31
                          and nu[1] * nu[2] < 2**31)
        self.fft_rev = (self.fft_lines and max(nu[0], nu[1]) > 1365 and nu[2] <= 65535
                        and (nf[0] + 31) // 32 <= 65535 and nu[2] * nf[0] < 2**31
                        and nu[2] * nu[1] < 2**31)
        # grid axis k holds axis ax[k]: the forward-order x pass writes whole
        # lines, x innermost, (n1, n2, n0)
        ax = [2, 1, 0] if self.fft_rev else ([1, 2, 0] if self.fft_lines else [0, 1, 2])
        self.grid_shape = [nu[a] for a in ax]

        # ---- targets: rescale, post factor, bin sort (device fp64) ----------
        stream = E.zstream_eligible(3, self.w2)
        self.bins_trg = (E.make_bins(3, self.w2, self.grid_shape, m=E.ZSTREAM_M) if stream else
                         E.make_bins(3, self.w2, self.grid_shape,
                                     cell_bytes=E.INTERP_CELL_BYTES, npts=self.M))
        hd = [2.0 * PI / nf for nf in self.nf]
        hg = [hd[d] * self.gam[d] for d in range(3)]
        h2 = [2.0 * PI / n for n in self.n_up]
        dq, fq = quadrature(self.beta, self.w)
        quad = torch.from_numpy(np.concatenate([dq, fq])).to(self.device)
        t_i1 = torch.empty((3, self.M), dtype=torch.int32, device=self.device)
        t_fr = torch.empty((3, self.M), dtype=torch.float32, device=self.device)
        t_key = torch.empty(self.M, dtype=torch.int32, device=self.device)
        post = torch.empty(self.M, dtype=torch.complex64, device=self.device)
        L.check(L.lib().mn_t3_setpts_trg(
            L.ctypes.byref(self.bins_trg), self.M, L.ptr3([s64[a] for a in ax]),
            L.d3([self.D[a] for a in ax]), L.d3([hg[a] for a in ax]), L.d3([h2[a] for a in ax]),
            L.d3([self.C[a] for a in ax]), self.isign, self._flags, L.ptr(quad), len(dq),
            L.ptr3([t_i1[d] for d in range(3)]), L.ptr3([t_fr[d] for d in range(3)]),
            L.ptr(t_key), L.ptr(post), L.stream()), "t3 targets")
        self.trg = E.SortedPoints(self.bins_trg, t_i1, t_fr, t_key, extra=post, stream=stream)
        del t_i1, t_fr, t_key, post
        # gather: direct per-target reads unless the targets are dense on the
        # grid (a staged tile per bin then serves many targets);
        # MN_T3_GATHER=direct|staged forces one
        gmode = os.environ.get("MN_T3_GATHER")
        if gmode not in (None, "direct", "staged"):
            raise ValueError(f"MN_T3_GATHER must be 'direct' or 'staged', not {gmode!r}")
        self.gather_direct = (gmode == "direct" or
                              (gmode is None and E.interp_direct_preferred(self.trg, self.w2,
                                                                           self.grid_shape)))

        # ---- mode deconvolution (-1)^|q| / phihat(2 pi q / n_up), q in
        # [-nf/2, nf/2); rocFFT's backward transform is unnormalised
        # (ref: gpu_t3.py:379-392).
        self.decs = []
        for d in range(3):
            q = np.arange(-self.nf[d] // 2, self.nf[d] // 2, dtype=np.float64)
            ph = kernel_ft(2.0 * PI * q / self.n_up[d], self.beta2, self.w2)
            self.decs.append(((-1.0) ** np.abs(q)) / ph)
        self.dev_dec = [torch.from_numpy(v.astype(np.float32)).to(self.device)
                        for v in self.decs]
        self.dev_dec64 = [torch.from_numpy(np.ascontiguousarray(v, dtype=np.float64))
                          .to(self.device) for v in self.decs]
        # spread: the tile spread (zero fill, atomic halo flushes) or the
        # owner-computes spread (bins of about 16^3 cells, each cell written
        # once), both accumulated on the matrix cores where their bins allow.
        # Measured on MI355X with uniform points (owner / tiles, ms), the
        # owner spread wins when taps per fine cell (P w^3 / prod nf) lie in
        # about [0.12, 45] on grids without a thin axis: 486^3 with 1e4 / 1e5
        # / 1e6 points 0.57 / 0.66 / 1.35 against 0.47 / 1.21 / 4.24; 300^3,
        # 1e6 (27 taps) 1.27 against 2.08; 240^3 (53) 1.47 against 1.20;
        # 180^3 (125) 1.69 against 0.56. Sparser grids favour the tiles' fast
        # zero fill, denser ones their single visit per point; thin slabs
        # (an axis of at most 18 cells) keep the LDS owner kernel and favour
        # the tiles (5760^2 x 18, 4e4 points: 4.9 against 2.3).
        # MN_T3_SPREAD=owner|tiles forces one.
        taps = float(self.P) * self.w ** 3 / float(np.prod([float(n) for n in self.nf]))
        mode = os.environ.get("MN_T3_SPREAD")
        if mode not in (None, "owner", "tiles"):
            raise ValueError(f"MN_T3_SPREAD must be 'owner' or 'tiles', not {mode!r}")
        self.spread_owner = (mode == "owner" or
                             (mode is None and 0.12 <= taps <= 45.0 and min(self.nf) > 18))
        if self.spread_owner:
            self.bins_src = E.owner_bins(self.w, self.nf)
        else:
            self.bins_src = E.t3_tile_bins(self.w, self.nf)
        self._hd = hd
        self._bf = None
        self._H = None
        self.low_mem = bool(low_mem) if low_mem is not None else False
        self.set_sources(x64)

    # ------------------------------------------------------------------
    def set_sources(self, x, backend="host"):
        """Per-frame source update against the frozen grid/target setup; new
        sources must lie inside the planned extent plus half the kernel guard
        band (else ValueError). Both backends run the same native-fp64 device
        setup. ref: gpu_t3.py:444-506."""
        if backend not in ("host", "gpu"):
            raise ValueError(f"unknown backend {backend!r}")
        x64 = [L.to_dev_f64(v, self.device) for v in x]
        P = x64[0].numel()
        if P < 1 or not all(v.numel() == P for v in x64):
            raise ValueError("source coordinate arrays must be non-empty, equal length")
        for d in range(3):
            lo, hi = self._xext[d]
            guard = 0.45 * (self.w + 1) * self.gam[d] * (2.0 * PI / self.nf[d])
            if float(x64[d].min()) < lo - guard or float(x64[d].max()) > hi + guard:
                raise ValueError(
                    f"set_sources: dim {d} sources exceed the frozen plan extent "
                    f"[{lo:.4g}, {hi:.4g}] (+guard {guard:.3g}); rebuild the plan for this "
                    "geometry")
        self.P = P
        i1 = torch.empty((3, P), dtype=torch.int32, device=self.device)
        fr = torch.empty((3, P), dtype=torch.float32, device=self.device)
        key = torch.empty(P, dtype=torch.int32, device=self.device)
        pre = torch.empty(P, dtype=torch.complex64, device=self.device)
        L.check(L.lib().mn_t3_setpts_src(
            L.ctypes.byref(self.bins_src), P, L.ptr3(x64), L.d3(self.C), L.d3(self.gam),
            L.d3(self._hd), L.d3(self.D), self.isign, self._flags,
            L.ptr3([i1[d] for d in range(3)]), L.ptr3([fr[d] for d in range(3)]), L.ptr(key),
            L.ptr(pre), L.stream()), "t3 sources")
        self.src = E.SortedPoints(self.bins_src, i1, fr, key, extra=pre, stream=self.spread_owner)

    @property
    def mx_perm(self):
        return self.src.perm

    @property
    def perm(self):
        return self.src.perm.cpu().numpy().astype(np.intp)

    def _buffers(self):
        if self._bf is None:
            nf, nu = self.nf, self.n_up
            self._bf = torch.empty(nf, dtype=torch.complex128, device=self.device)
            self._H = torch.empty(self.grid_shape, dtype=torch.complex64, device=self.device)
            c128 = dict(dtype=torch.complex128, device=self.device)
            if self.fft_rev:
                self._T = (torch.empty((nu[2], nf[0], nf[1]), **c128),
                           torch.empty((nu[2], nf[0], nu[1]), **c128),
                           torch.empty((nu[2], nu[1], nf[0]), **c128))
                self._H64 = None
            elif self.fft_lines:
                self._T = (torch.empty((nf[0], nf[1], nu[2]), **c128),
                           torch.empty((nf[0], nu[1], nu[2]), **c128))
                self._H64 = None
            else:
                self._T = None
                self._H64 = torch.empty(nu, dtype=torch.complex128, device=self.device)
        return self._bf, self._H, self._H64

    def _inner_fft(self, bf, H, H64, tm):
        """H = (complex64) FFT(pad(bf * dec0 x dec1 x dec2)) on the n_up grid."""
        nf, nu, d = self.nf, self.n_up, self.dev_dec64
        if self.fft_rev:
            T1, T2, T3 = self._T
            with tm("fft"):
                # z lines -> (n2, nf0, nf1); y lines -> (n2, nf0, n1); transpose
                # -> (n2, n1, nf0); x lines -> H (n2, n1, n0)
                E.fft64_lines(nf[0] * nf[1], nf[2], 1, nu[2], self.isign, bf, d[2], T1,
                              layout="lines_last")
                E.fft64_lines(nu[2] * nf[0], nf[1], 1, nu[1], self.isign, T1, d[1], T2)
                E.transpose_c128(nu[2], nf[0], nu[1], T2, T3)
                E.fft64_lines(nu[2] * nu[1], nf[0], 1, nu[0], self.isign, T3, d[0], H)
            return
        if self.fft_lines:
            T1, T2 = self._T
            with tm("fft"):
                # z lines -> (nf0, nf1, n2); y lines -> (nf0, n1, n2); x lines
                # -> H (n1, n2, n0), each x line stored whole: 2.31 against
                # 2.55 ms for the x pass at 640^3 when the strided x lines
                # were stored in place (runs of 4 complex64 values)
                E.fft64_lines(nf[0] * nf[1], nf[2], 1, nu[2], self.isign, bf, d[2], T1)
                E.fft64_lines(nf[0], nf[1], nu[2], nu[1], self.isign, T1, d[1], T2)
                E.fft64_lines(1, nf[0], nu[1] * nu[2], nu[0], self.isign, T2, d[0], H,
                              layout="lines_first")
            return
        with tm("pad+deconv"):
            E.pad_deconv_c128(self.n_up, self.nf, bf, d, H64)
        with tm("fft"):
            E.fft_f64(H64, self.n_up, self.isign)
            E.round_c64(H64, H)

    def _run(self, cd, tm):
        """Spread (fp64 products and accumulation into a complex128 grid),
        pad + deconvolve and FFT in fp64, round to complex64, gather with the
        post factor. The mode deconvolution and the target deconvolution
        1/phihat(theta) amplify white rounding noise of the inner grid at the
        band edges, so everything up to the FFT output is fp64 (at 1e6 x 1e6
        points, eps 1e-5: fp32 spread products and FFT give 7.5e-5 relative
        error, this path about the fp64 reference's 1.4e-5)."""
        bf, H, H64 = self._buffers()
        out = torch.empty(self.M, dtype=torch.complex64, device=self.device)
        with tm("spread"):
            if self.spread_owner:
                E.spread_owner_c128(self.src, self.beta, cd, bf, pre=self.src.extra)
            else:
                E.spread_c128(self.src, self.beta, cd, bf, pre=self.src.extra)
        self._inner_fft(bf, H, H64, tm)
        with tm("gather"):
            if self.gather_direct:
                E.interp_direct(self.trg, self.beta2, H, out, post=self.trg.extra)
            else:
                E.interp(self.trg, self.beta2, H, out, post=self.trg.extra)
        if self.low_mem:
            self._bf = self._H = self._H64 = self._T = None
        return out

    def _strengths(self, c):
        cd = L.to_dev_c64(c, self.device).reshape(-1)
        if cd.numel() != self.P:
            raise PlanArgumentError(f"c.size ({cd.numel()}) must equal number of sources "
                                    f"({self.P})")
        return cd

    def execute(self, c, return_np=True):
        """ref: gpu_t3.py:1287-1349."""
        tm = E.StageTimer(self.profile)
        out = self._run(self._strengths(c), tm)
        if self.profile:
            self.last_profile = tm.times_ms()
        return L.to_host(out) if return_np else out

    def execute_batch(self, cs, return_np=True):
        """nch strength channels through one plan: (nch, P) -> (nch, M).
        ref: gpu_t3.py:941-1041 (the reference supports it in slab mode only;
        here every plan supports it)."""
        cs_t = cs if isinstance(cs, torch.Tensor) else np.asarray(cs)
        if cs_t.ndim != 2 or cs_t.shape[1] != self.P:
            raise ValueError(f"cs must have shape (nch, {self.P})")
        cd = L.to_dev_c64(cs_t, self.device)
        tm = E.StageTimer(False)
        res = torch.stack([self._run(cd[ch], tm) for ch in range(cd.shape[0])])
        return L.to_host(res) if return_np else res

    def execute_profiled(self, c):
        """(result, {stage: seconds}) with HIP-event stage times; the prephase
        is fused into the spread and, on the line-FFT path, pad+deconv into
        the fft (ref: gpu_t3.py:1351-1364)."""
        tm = E.StageTimer(True)
        out = self._run(self._strengths(c), tm)
        ms = tm.times_ms()
        times = {"prephase": 0.0, "spread": 0.0, "pad+deconv": 0.0}
        times.update({k: v / 1e3 for k, v in ms.items()})
        return L.to_host(out), times
