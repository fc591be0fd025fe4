"""finufft-compatible API (drop-in mirror of the reference's surface).

    import mlx_nufft_amd as finufft
    fk = finufft.nufft2d1(x, y, c, (N1, N2), eps=1e-6)
    plan = finufft.Plan(1, (N1, N2), n_trans=8, eps=1e-6)
    plan.setpts(x, y)
    fk = plan.execute(c)

Semantics follow the reference (ref: mlx_nufft/api.py:1-388), itself a
mirror of finufft 2.x: modeord=0 mode boxes (even or odd N), isign >= 0
means +i (type 1/3 default +1, type 2 default -1), a leading n_trans axis
on strengths/modes, out= filled in place and returned, complex128 in ->
complex128 out, eps below 1e-6 clamped with a warning, modeord=1 raises
NotImplementedError, 1D/2D type 3 run as degenerate 3D type 3.

Plan.execute with n_trans > 1 runs one batched spread + batched FFT for
type 1 (the reference loops single transforms, api.py:342).
"""

import warnings

import numpy as np
import torch

from .nd import Type1PlanND, Type2PlanND
from .t3 import GpuT3Plan

_EPS_FLOOR = 1e-6
_IGNORED_OPTS = {
    "nthreads", "debug", "spread_debug", "showwarn", "fftw", "spread_sort",
    "spread_kerevalmeth", "spread_kerpad", "chkbnds", "maxbatchsize",
    "spread_thread", "spread_nthr_atomic", "spread_max_sp_size",
}


def _check_opts(kwargs):
    """ref: api.py:47-61."""
    opts = dict(kwargs)
    if opts.pop("modeord", 0) not in (0,):
        raise NotImplementedError("modeord=1 (FFT ordering) not implemented")
    upsampfac = opts.pop("upsampfac", None)
    if upsampfac in (0, 0.0):
        upsampfac = None
    prec = opts.pop("prec", "crit64")
    fft_backend = opts.pop("fft_backend", "mlx")
    for k in list(opts):
        if k in _IGNORED_OPTS:
            opts.pop(k)
    if opts:
        warnings.warn(f"mlx-nufft: ignoring unknown options {sorted(opts)}")
    return upsampfac, prec, fft_backend


def _norm_eps(eps):
    """ref: api.py:64-71."""
    eps = float(eps)
    if eps < _EPS_FLOOR:
        warnings.warn(f"mlx-nufft: eps={eps:g} is below the fp32 pipeline floor; clamping to "
                      f"{_EPS_FLOOR:g}")
        eps = _EPS_FLOOR
    return eps


def _norm_isign(isign, default):
    if isign is None:
        return default
    return +1 if isign >= 0 else -1


def _np(a):
    return a.detach().cpu().numpy() if isinstance(a, torch.Tensor) else np.asarray(a)


def _out_dtype(*arrays):
    """ref: api.py:80-84."""
    for a in arrays:
        dt = a.dtype if isinstance(a, torch.Tensor) else np.asarray(a).dtype
        if dt in (np.complex128, np.float64, torch.complex128, torch.float64):
            return np.complex128
    return np.complex64


def _vec_shape(data, inner_ndim, inner_shape=None):
    """Split into (n_trans, stacked data); strict trailing-shape check.
    ref: api.py:87-102."""
    data = _np(data)
    if data.ndim == inner_ndim:
        out = 1, data[None, ...]
    elif data.ndim == inner_ndim + 1:
        out = data.shape[0], data
    else:
        raise ValueError(f"data must have {inner_ndim} or {inner_ndim + 1} dims, got shape "
                         f"{data.shape}")
    if inner_shape is not None and out[1].shape[1:] != tuple(inner_shape):
        raise ValueError(f"data inner shape {out[1].shape[1:]} must be {tuple(inner_shape)}")
    return out


def _fill_out(out, res, dtype):
    """ref: api.py:105-115."""
    res = res.astype(dtype, copy=False)
    if out is not None:
        if out.shape != res.shape and out.shape != (1,) + res.shape \
                and (1,) + out.shape != res.shape:
            raise ValueError(f"out.shape {out.shape} does not match result shape {res.shape}")
        np.copyto(out, res.reshape(out.shape))
        return out
    return res


def _embed3(arrs, dim):
    """Zero-pad a dim<3 coordinate tuple to 3 components (ref: api.py:118-122)."""
    arrs = [_np(a).astype(np.float64).ravel() for a in arrs]
    z = np.zeros(arrs[0].size)
    return tuple(arrs) + (z,) * (3 - dim)


def _modes_tuple(n_modes, dim, out, out_offset=0):
    """ref: api.py:125-135."""
    if n_modes is None:
        if out is None:
            raise ValueError("either n_modes or out must be supplied")
        shape = out.shape[out_offset:]
        if len(shape) != dim:
            raise ValueError(f"out shape {out.shape} does not match dim {dim}")
        return tuple(int(n) for n in shape)
    if np.isscalar(n_modes):
        return (int(n_modes),) * dim
    return tuple(int(n) for n in n_modes)


def _warn_no_vkfft(fft_backend, what):
    if fft_backend != "mlx":
        warnings.warn(f"mlx-nufft: fft_backend={fft_backend!r} applies only to 3D type-3 "
                      f"(slab); ignored for {what}")


def _t1_run(plan, cv, n_tr):
    if n_tr == 1:
        return plan.execute(cv[0])[None]
    return plan.execute_batch(cv)


# ---------------------------------------------------------------------------
# type 1


def _nufft_t1(dim, coords, c, n_modes, out, eps, isign, kwargs):
    """ref: api.py:148-164."""
    upsampfac, prec, fft_backend = _check_opts(kwargs)
    _warn_no_vkfft(fft_backend, "type-1")
    eps = _norm_eps(eps)
    isign = _norm_isign(isign, +1)
    dtype = _out_dtype(c)
    M = _np(coords[0]).size
    n_tr, cv = _vec_shape(c, 1, inner_shape=(M,))
    if out is not None and n_modes is None:
        n_modes = _modes_tuple(None, dim, out, out_offset=(1 if n_tr > 1 else 0))
    N = _modes_tuple(n_modes, dim, out)
    kw = {} if upsampfac is None else {"upsampfac": upsampfac}
    plan = Type1PlanND(coords, N, eps=eps, isign=isign, prec=prec, **kw)
    res = _t1_run(plan, cv, n_tr)
    if n_tr == 1 and _np(c).ndim == 1:
        res = res[0]
    return _fill_out(out, res, dtype)


def nufft1d1(x, c, n_modes=None, out=None, eps=1e-6, isign=1, **kwargs):
    """1D type-1: f[k] = sum_j c[j] exp(+/-i k x(j))."""
    return _nufft_t1(1, (x,), c, n_modes, out, eps, isign, kwargs)


def nufft2d1(x, y, c, n_modes=None, out=None, eps=1e-6, isign=1, **kwargs):
    """2D type-1: f[k1,k2] = sum_j c[j] exp(+/-i (k1 x(j) + k2 y(j)))."""
    return _nufft_t1(2, (x, y), c, n_modes, out, eps, isign, kwargs)


def nufft3d1(x, y, z, c, n_modes=None, out=None, eps=1e-6, isign=1, **kwargs):
    """3D type-1: f[k1,k2,k3] = sum_j c[j] exp(+/-i k . x_j)."""
    return _nufft_t1(3, (x, y, z), c, n_modes, out, eps, isign, kwargs)


# ---------------------------------------------------------------------------
# type 2


def _nufft_t2(dim, coords, f, out, eps, isign, kwargs):
    """ref: api.py:186-199."""
    upsampfac, prec, fft_backend = _check_opts(kwargs)
    _warn_no_vkfft(fft_backend, "type-2")
    eps = _norm_eps(eps)
    isign = _norm_isign(isign, -1)
    dtype = _out_dtype(f)
    n_tr, fv = _vec_shape(f, dim)
    N = fv.shape[1:]
    kw = {} if upsampfac is None else {"upsampfac": upsampfac}
    plan = Type2PlanND(coords, N, eps=eps, isign=isign, prec=prec, **kw)
    res = np.stack([plan.execute(fv[t]) for t in range(n_tr)])
    if n_tr == 1 and _np(f).ndim == dim:
        res = res[0]
    return _fill_out(out, res, dtype)


def nufft1d2(x, f, out=None, eps=1e-6, isign=-1, **kwargs):
    """1D type-2: c[j] = sum_k f[k] exp(+/-i k x(j))."""
    return _nufft_t2(1, (x,), f, out, eps, isign, kwargs)


def nufft2d2(x, y, f, out=None, eps=1e-6, isign=-1, **kwargs):
    """2D type-2: c[j] = sum_{k1,k2} f[k1,k2] exp(+/-i (k1 x(j) + k2 y(j)))."""
    return _nufft_t2(2, (x, y), f, out, eps, isign, kwargs)


def nufft3d2(x, y, z, f, out=None, eps=1e-6, isign=-1, **kwargs):
    """3D type-2: c[j] = sum_k f[k] exp(+/-i k . x_j)."""
    return _nufft_t2(3, (x, y, z), f, out, eps, isign, kwargs)


# ---------------------------------------------------------------------------
# type 3


def _nufft_t3(dim, src, c, trg, out, eps, isign, kwargs):
    """ref: api.py:221-236."""
    upsampfac, prec, fft_backend = _check_opts(kwargs)
    if upsampfac is not None and upsampfac != 1.25:
        warnings.warn("mlx-nufft: type-3 runs the validated sigma=1.25 pipeline; "
                      "upsampfac ignored")
    eps = _norm_eps(eps)
    isign = _norm_isign(isign, +1)
    dtype = _out_dtype(c)
    M = _np(src[0]).size
    n_tr, cv = _vec_shape(c, 1, inner_shape=(M,))
    plan = GpuT3Plan(_embed3(src, dim), _embed3(trg, dim), eps=eps, isign=isign, prec=prec,
                     fft_backend=fft_backend)
    res = np.stack([plan.execute(cv[t]) for t in range(n_tr)])
    if n_tr == 1 and _np(c).ndim == 1:
        res = res[0]
    return _fill_out(out, res, dtype)


def nufft1d3(x, c, s, out=None, eps=1e-6, isign=1, **kwargs):
    """1D type-3: f[k] = sum_j c[j] exp(+/-i s[k] x[j])."""
    return _nufft_t3(1, (x,), c, (s,), out, eps, isign, kwargs)


def nufft2d3(x, y, c, s, t, out=None, eps=1e-6, isign=1, **kwargs):
    """2D type-3: f[k] = sum_j c[j] exp(+/-i (s[k] x[j] + t[k] y[j]))."""
    return _nufft_t3(2, (x, y), c, (s, t), out, eps, isign, kwargs)


def nufft3d3(x, y, z, c, s, t, u, out=None, eps=1e-6, isign=1, **kwargs):
    """3D type-3: f[k] = sum_j c[j] exp(+/-i (s,t,u)_k . (x,y,z)_j)."""
    return _nufft_t3(3, (x, y, z), c, (s, t, u), out, eps, isign, kwargs)


# ---------------------------------------------------------------------------
# Plan interface


class Plan:
    """finufft.Plan-compatible plan/setpts/execute interface.

    Plan(nufft_type, n_modes_or_dim, n_trans=1, eps=1e-6, isign=None,
         dtype='complex128', **kwargs)
    ref: api.py:258-388.
    """

    def __init__(self, nufft_type, n_modes_or_dim, n_trans=1, eps=1e-6, isign=None,
                 dtype="complex128", **kwargs):
        if nufft_type not in (1, 2, 3):
            raise ValueError("nufft_type must be 1, 2 or 3")
        self.type = int(nufft_type)
        self.n_trans = int(n_trans)
        self.eps = _norm_eps(eps)
        self.isign = _norm_isign(isign, -1 if self.type == 2 else +1)
        self.dtype = np.dtype(dtype)
        if self.dtype not in (np.complex64, np.complex128):
            raise ValueError("dtype must be complex64 or complex128")
        self._upsampfac, self._prec, self._fft_backend = _check_opts(kwargs)
        if self._fft_backend != "mlx" and self.type != 3:
            _warn_no_vkfft(self._fft_backend, f"type-{self.type}")
            self._fft_backend = "mlx"
        if self.type == 3:
            self.dim = int(n_modes_or_dim)
            self.n_modes = None
        else:
            if np.isscalar(n_modes_or_dim):
                n_modes_or_dim = (n_modes_or_dim,)
            self.n_modes = tuple(int(n) for n in n_modes_or_dim)
            self.dim = len(self.n_modes)
        if self.dim not in (1, 2, 3):
            raise ValueError("dim must be 1, 2 or 3")
        self._plan = None
        self._adjoint = None
        self._n_targets = None

    def setpts(self, x=None, y=None, z=None, s=None, t=None, u=None):
        coords = [v for v in (x, y, z) if v is not None]
        if len(coords) != self.dim:
            raise ValueError(f"expected {self.dim} coordinate arrays, got {len(coords)}")
        kw = {} if self._upsampfac is None else {"upsampfac": self._upsampfac}
        self._adjoint = None
        if self.type == 1:
            self._plan = Type1PlanND(tuple(coords), self.n_modes, eps=self.eps, isign=self.isign,
                                     prec=self._prec, **kw)
        elif self.type == 2:
            self._plan = Type2PlanND(tuple(coords), self.n_modes, eps=self.eps, isign=self.isign,
                                     prec=self._prec, **kw)
        else:
            if self._upsampfac is not None and self._upsampfac != 1.25:
                warnings.warn("mlx-nufft: type-3 runs the validated sigma=1.25 pipeline; "
                              "upsampfac ignored")
            trg = [v for v in (s, t, u) if v is not None]
            if len(trg) != self.dim:
                raise ValueError(f"expected {self.dim} target arrays, got {len(trg)}")
            self._plan = GpuT3Plan(_embed3(coords, self.dim), _embed3(trg, self.dim),
                                   eps=self.eps, isign=self.isign, prec=self._prec,
                                   fft_backend=self._fft_backend)
            self._n_targets = _np(trg[0]).size
        self._coords = [_np(v) for v in coords]
        self._targets = None if self.type != 3 else [_np(v) for v in (s, t, u) if v is not None]

    def execute(self, data, out=None):
        if self._plan is None:
            raise RuntimeError("setpts() must be called before execute()")
        if self.type == 2:
            inner, ishape = self.dim, self.n_modes
        else:
            inner, ishape = 1, (self._plan.P,)
        n_tr, dv = _vec_shape(data, inner, inner_shape=ishape)
        if n_tr != self.n_trans:
            raise ValueError(f"data has {n_tr} vectors, plan has n_trans={self.n_trans}")
        if self.type == 1:
            res = _t1_run(self._plan, dv, n_tr)
        else:
            res = np.stack([self._plan.execute(dv[k]) for k in range(self.n_trans)])
        if self.n_trans == 1 and _np(data).ndim == inner:
            res = res[0]
        return _fill_out(out, res, self.dtype)

    def execute_adjoint(self, data, out=None):
        """Adjoint of the planned transform: the sibling transform with isign
        negated (type 1 <-> type 2; type 3 with sources and targets swapped).
        ref: api.py:347-388."""
        if self._plan is None:
            raise RuntimeError("setpts() must be called before execute_adjoint()")
        if self._adjoint is None:
            kw = {} if self._upsampfac is None else {"upsampfac": self._upsampfac}
            if self.type == 1:
                self._adjoint = Type2PlanND(tuple(self._coords), self.n_modes, eps=self.eps,
                                            isign=-self.isign, prec=self._prec, **kw)
            elif self.type == 2:
                self._adjoint = Type1PlanND(tuple(self._coords), self.n_modes, eps=self.eps,
                                            isign=-self.isign, prec=self._prec, **kw)
            else:
                self._adjoint = GpuT3Plan(_embed3(self._targets, self.dim),
                                          _embed3(self._coords, self.dim), eps=self.eps,
                                          isign=-self.isign, prec=self._prec,
                                          fft_backend=self._fft_backend)
        if self.type == 1:
            inner, ishape = self.dim, self.n_modes
        elif self.type == 2:
            inner, ishape = 1, (self._plan.P,)
        else:
            inner, ishape = 1, (self._n_targets,)
        n_tr, dv = _vec_shape(data, inner, inner_shape=ishape)
        if n_tr != self.n_trans:
            raise ValueError(f"data has {n_tr} vectors, plan has n_trans={self.n_trans}")
        if self.type == 2:
            res = _t1_run(self._adjoint, dv, n_tr)
        else:
            res = np.stack([self._adjoint.execute(dv[k]) for k in range(self.n_trans)])
        if self.n_trans == 1 and _np(data).ndim == inner:
            res = res[0]
        return _fill_out(out, res, self.dtype)
