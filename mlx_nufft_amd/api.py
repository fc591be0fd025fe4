"""finufft-style functional and Plan surface over the engine's plans.

    import mlx_nufft_amd as finufft
    fk = finufft.nufft2d1(x, y, c, (N1, N2), eps=1e-6)
    plan = finufft.Plan(1, (N1, N2), n_trans=8, eps=1e-6)
    plan.setpts(x, y)
    fk = plan.execute(c)

The public names, signatures, defaults, option keywords and exception
classes are the reference's interface (ref: mlx_nufft/api.py:167-388), which
mirrors finufft 2.x: modeord=0 mode boxes (even or odd N); isign >= 0 means
+i (type 1 and 3 default +1, type 2 default -1); a leading n_trans axis on
strengths and mode arrays; out= filled in place and returned; complex128 or
float64 data in gives complex128 out; eps below 1e-6 is raised to 1e-6 with
a warning (the fp32 pipeline's floor); modeord=1 raises
NotImplementedError; 1D and 2D type 3 run as 3D type 3 with zero
coordinates on the missing axes.

Below that interface the module is organised around three pieces:
- `_Options`, the keyword options parsed once per call or plan;
- `_KINDS`, one entry per transform type saying how it builds an engine
  plan, what data it takes, how it runs n vectors and what its adjoint is;
- `_deliver`, which turns the stacked device result into the caller's
  array (dtype, squeezed single vector, out=).
Many vectors run as one batched engine call where the engine has one
(type-1 execute_batch, type-3 execute_batch); the reference loops.
"""

import warnings
from dataclasses import dataclass

import numpy as np
import torch

from .nd import Type1PlanND, Type2PlanND
from .t3 import GpuT3Plan

_MIN_EPS = 1e-6

# finufft options that tune its CPU library (threads, sorting and kernel
# evaluation heuristics, debug output). They have no meaning here and are
# accepted silently, as the reference does.
_CPU_LIBRARY_OPTIONS = frozenset((
    "nthreads", "debug", "spread_debug", "showwarn", "fftw", "spread_sort",
    "spread_kerevalmeth", "spread_kerpad", "chkbnds", "maxbatchsize", "spread_thread",
    "spread_nthr_atomic", "spread_max_sp_size",
))


@dataclass(frozen=True)
class _Options:
    """Keyword options of one call or plan, after validation."""

    eps: float
    upsampfac: object   # None: the engine plan's own default
    prec: str
    fft_backend: str

    @classmethod
    def parse(cls, eps, kwargs):
        opts = dict(kwargs)
        if opts.pop("modeord", 0) != 0:
            raise NotImplementedError("modeord=1 (FFT-ordered modes) is not supported; "
                                      "use modeord=0")
        sigma = opts.pop("upsampfac", None)
        if sigma == 0:
            sigma = None   # finufft's "choose for me"
        prec = opts.pop("prec", "crit64")
        backend = opts.pop("fft_backend", "mlx")
        unknown = sorted(k for k in opts if k not in _CPU_LIBRARY_OPTIONS)
        if unknown:
            warnings.warn(f"mlx_nufft_amd: unrecognised options {unknown} have no effect")
        eps = float(eps)
        if eps < _MIN_EPS:
            warnings.warn(f"mlx_nufft_amd: eps={eps:g} lies below what the fp32 pipeline "
                          f"can deliver; running at eps={_MIN_EPS:g}")
            eps = _MIN_EPS
        return cls(eps, sigma, prec, backend)

    def sigma_kw(self):
        return {} if self.upsampfac is None else {"upsampfac": self.upsampfac}


def _sign(isign, default):
    if isign is None:
        return default
    return 1 if isign >= 0 else -1


def _is_wide(a):
    """complex128/float64 data asks for complex128 results."""
    dt = a.dtype if isinstance(a, torch.Tensor) else np.asarray(a).dtype
    return dt in (np.complex128, np.float64, torch.complex128, torch.float64)


def _ndim(a):
    return a.dim() if isinstance(a, torch.Tensor) else np.ndim(a)


def _shape(a):
    return tuple(a.shape) if isinstance(a, torch.Tensor) else np.shape(a)


def _size(a):
    return a.numel() if isinstance(a, torch.Tensor) else np.size(a)


def _host_f64(a):
    if isinstance(a, torch.Tensor):
        a = a.detach().cpu().numpy()
    return np.asarray(a, dtype=np.float64).ravel()


def _as_3d(coords, dim):
    """Coordinates of a dim < 3 type-3 problem as 3 arrays (zeros appended)."""
    arrs = [_host_f64(a) for a in coords]
    return tuple(arrs) + tuple(np.zeros(arrs[0].size) for _ in range(3 - dim))


def _vectors(data, rank, inner=None):
    """data as (n, single): n vectors of `rank` dims each; single says the
    caller passed one unstacked vector. The inner shape must equal `inner`
    when given (no silent truncation)."""
    nd = _ndim(data)
    if nd == rank:
        n, single = 1, True
        shape = _shape(data)
    elif nd == rank + 1:
        n, single = _shape(data)[0], False
        shape = _shape(data)[1:]
    else:
        raise ValueError(f"expected data with {rank} dims (one vector) or {rank + 1} "
                         f"(a stack of vectors); got shape {_shape(data)}")
    if inner is not None and tuple(shape) != tuple(inner):
        raise ValueError(f"each data vector must have shape {tuple(inner)}, got "
                         f"{tuple(shape)}")
    return int(n), single


def _stack_view(data, rank):
    """data with a leading vector axis (a view when possible)."""
    if _ndim(data) == rank:
        return data[None] if isinstance(data, torch.Tensor) else np.asarray(data)[None]
    return data if isinstance(data, torch.Tensor) else np.asarray(data)


def _deliver(res, single, dtype, out):
    """Device result (n, ...) -> the caller's array: one D2H copy, squeezed
    for a single vector, cast to dtype, copied into out= when given (and out
    itself returned)."""
    host = res.detach().cpu().numpy()
    if single:
        host = host[0]
    host = host.astype(dtype, copy=False)
    if out is None:
        return host
    oshape = tuple(out.shape)
    if oshape not in (host.shape, (1,) + host.shape) and (1,) + oshape != host.shape:
        raise ValueError(f"out has shape {oshape}; the result has shape {host.shape}")
    np.copyto(out, host.reshape(oshape))
    return out


# ---------------------------------------------------------------------------
# The three transform kinds


class _Type1:
    """Nonuniform points -> modes."""

    code = 1
    default_isign = +1
    adjoint_code = 2

    @staticmethod
    def rank(dim):
        return 1

    @staticmethod
    def build(dim, coords, targets, n_modes, opts, isign):
        if opts.fft_backend != "mlx":
            _warn_backend(opts.fft_backend, "type 1")
        return Type1PlanND(tuple(coords), n_modes, eps=opts.eps, isign=isign, prec=opts.prec,
                           **opts.sigma_kw())

    @staticmethod
    def inner(plan, n_modes):
        return (plan.P,)

    @staticmethod
    def run(plan, stack, n):
        if n == 1:
            return plan.execute(stack[0], return_np=False)[None]
        return plan.execute_batch(stack, return_np=False)


class _Type2:
    """Modes -> nonuniform points."""

    code = 2
    default_isign = -1
    adjoint_code = 1

    @staticmethod
    def rank(dim):
        return dim

    @staticmethod
    def build(dim, coords, targets, n_modes, opts, isign):
        if opts.fft_backend != "mlx":
            _warn_backend(opts.fft_backend, "type 2")
        return Type2PlanND(tuple(coords), n_modes, eps=opts.eps, isign=isign, prec=opts.prec,
                           **opts.sigma_kw())

    @staticmethod
    def inner(plan, n_modes):
        return tuple(n_modes)

    @staticmethod
    def run(plan, stack, n):
        return torch.stack([plan.execute(stack[k], return_np=False) for k in range(n)])


class _Type3:
    """Nonuniform sources -> nonuniform targets."""

    code = 3
    default_isign = +1
    adjoint_code = 3

    @staticmethod
    def rank(dim):
        return 1

    @staticmethod
    def build(dim, coords, targets, n_modes, opts, isign):
        if opts.upsampfac is not None and opts.upsampfac != 1.25:
            warnings.warn("mlx_nufft_amd: type 3 always runs at upsampfac=1.25; the "
                          "requested value has no effect")
        return GpuT3Plan(_as_3d(coords, dim), _as_3d(targets, dim), eps=opts.eps, isign=isign,
                         prec=opts.prec, fft_backend=opts.fft_backend)

    @staticmethod
    def inner(plan, n_modes):
        return (plan.P,)

    @staticmethod
    def run(plan, stack, n):
        if n == 1:
            return plan.execute(stack[0], return_np=False)[None]
        return plan.execute_batch(stack, return_np=False)


_KINDS = {1: _Type1, 2: _Type2, 3: _Type3}


def _warn_backend(backend, what):
    warnings.warn(f"mlx_nufft_amd: fft_backend={backend!r} only concerns 3D type 3; "
                  f"{what} uses the built-in FFT")


def _modes_from_out(out, dim, stacked):
    shape = tuple(out.shape)[1 if stacked else 0:]
    if len(shape) != dim:
        raise ValueError(f"out has shape {tuple(out.shape)}, which holds no {dim}D mode box")
    return tuple(int(n) for n in shape)


def _mode_box(n_modes, dim):
    if np.isscalar(n_modes):
        return (int(n_modes),) * dim
    return tuple(int(n) for n in n_modes)


def _oneshot(code, dim, coords, data, targets, n_modes, out, eps, isign, kwargs):
    """Plan, run and deliver one finufft-style call."""
    kind = _KINDS[code]
    opts = _Options.parse(eps, kwargs)
    sign = _sign(isign, kind.default_isign)
    wide = _is_wide(data)
    rank = kind.rank(dim)
    if code == 2:
        n, single = _vectors(data, rank)
        n_modes = _shape(data)[-dim:]
    else:
        n, single = _vectors(data, rank, inner=(_size(coords[0]),))
        if code == 1:
            if n_modes is None:
                if out is None:
                    raise ValueError("type 1 needs n_modes, or out= to take the mode box from")
                n_modes = _modes_from_out(out, dim, stacked=n > 1)
            n_modes = _mode_box(n_modes, dim)
    plan = kind.build(dim, coords, targets, n_modes, opts, sign)
    res = kind.run(plan, _stack_view(data, rank), n)
    return _deliver(res, single, np.complex128 if wide else np.complex64, out)


# ---------------------------------------------------------------------------
# finufft-style functions (signatures and defaults: ref api.py:167-251)


def nufft1d1(x, c, n_modes=None, out=None, eps=1e-6, isign=1, **kwargs):
    """1D type 1: f[k] = sum_j c[j] exp(+/-i k x[j])."""
    return _oneshot(1, 1, (x,), c, None, n_modes, out, eps, isign, kwargs)


def nufft2d1(x, y, c, n_modes=None, out=None, eps=1e-6, isign=1, **kwargs):
    """2D type 1: f[k1,k2] = sum_j c[j] exp(+/-i (k1 x[j] + k2 y[j]))."""
    return _oneshot(1, 2, (x, y), c, None, n_modes, out, eps, isign, kwargs)


def nufft3d1(x, y, z, c, n_modes=None, out=None, eps=1e-6, isign=1, **kwargs):
    """3D type 1: f[k] = sum_j c[j] exp(+/-i k . (x[j], y[j], z[j]))."""
    return _oneshot(1, 3, (x, y, z), c, None, n_modes, out, eps, isign, kwargs)


def nufft1d2(x, f, out=None, eps=1e-6, isign=-1, **kwargs):
    """1D type 2: c[j] = sum_k f[k] exp(+/-i k x[j])."""
    return _oneshot(2, 1, (x,), f, None, None, out, eps, isign, kwargs)


def nufft2d2(x, y, f, out=None, eps=1e-6, isign=-1, **kwargs):
    """2D type 2: c[j] = sum_{k1,k2} f[k1,k2] exp(+/-i (k1 x[j] + k2 y[j]))."""
    return _oneshot(2, 2, (x, y), f, None, None, out, eps, isign, kwargs)


def nufft3d2(x, y, z, f, out=None, eps=1e-6, isign=-1, **kwargs):
    """3D type 2: c[j] = sum_k f[k] exp(+/-i k . (x[j], y[j], z[j]))."""
    return _oneshot(2, 3, (x, y, z), f, None, None, out, eps, isign, kwargs)


def nufft1d3(x, c, s, out=None, eps=1e-6, isign=1, **kwargs):
    """1D type 3: f[k] = sum_j c[j] exp(+/-i s[k] x[j])."""
    return _oneshot(3, 1, (x,), c, (s,), None, out, eps, isign, kwargs)


def nufft2d3(x, y, c, s, t, out=None, eps=1e-6, isign=1, **kwargs):
    """2D type 3: f[k] = sum_j c[j] exp(+/-i (s[k] x[j] + t[k] y[j]))."""
    return _oneshot(3, 2, (x, y), c, (s, t), None, out, eps, isign, kwargs)


def nufft3d3(x, y, z, c, s, t, u, out=None, eps=1e-6, isign=1, **kwargs):
    """3D type 3: f[k] = sum_j c[j] exp(+/-i (s[k], t[k], u[k]) . (x[j], y[j], z[j]))."""
    return _oneshot(3, 3, (x, y, z), c, (s, t, u), None, out, eps, isign, kwargs)


# ---------------------------------------------------------------------------
# Plan (ref api.py:258-388)


class Plan:
    """finufft.Plan-style interface: Plan(type, n_modes_or_dim, ...), then
    setpts(...) once per point set and execute(...) per data stack.

    For types 1 and 2, n_modes_or_dim is the mode box (its length is the
    dimension); for type 3 it is the dimension. setpts builds the engine
    plan (point setup and sort run there); execute runs n_trans vectors
    through it, and execute_adjoint runs the adjoint transform (built on
    first use and kept until the next setpts).
    """

    def __init__(self, nufft_type, n_modes_or_dim, n_trans=1, eps=1e-6, isign=None,
                 dtype="complex128", **kwargs):
        if nufft_type not in _KINDS:
            raise ValueError(f"nufft_type must be 1, 2 or 3, got {nufft_type!r}")
        self._kind = _KINDS[nufft_type]
        self.type = self._kind.code
        self.n_trans = int(n_trans)
        self.dtype = np.dtype(dtype)
        if self.dtype not in (np.complex64, np.complex128):
            raise ValueError(f"dtype must be complex64 or complex128, got {self.dtype}")
        self._opts = _Options.parse(eps, kwargs)
        self.eps = self._opts.eps
        self.isign = _sign(isign, self._kind.default_isign)
        if self.type == 3:
            self.dim, self.n_modes = int(n_modes_or_dim), None
        else:
            box = (n_modes_or_dim,) if np.isscalar(n_modes_or_dim) else n_modes_or_dim
            self.n_modes = tuple(int(n) for n in box)
            self.dim = len(self.n_modes)
            if self._opts.fft_backend != "mlx":
                _warn_backend(self._opts.fft_backend, f"type {self.type}")
                self._opts = _Options(self._opts.eps, self._opts.upsampfac, self._opts.prec,
                                      "mlx")
        if self.dim not in (1, 2, 3):
            raise ValueError(f"the dimension must be 1, 2 or 3, got {self.dim}")
        self._plan = None
        self._adjoint = None
        self._points = None    # source coordinates of the current setpts
        self._targets = None   # type-3 target coordinates

    def setpts(self, x=None, y=None, z=None, s=None, t=None, u=None):
        pts = tuple(v for v in (x, y, z) if v is not None)
        if len(pts) != self.dim:
            raise ValueError(f"a {self.dim}D plan takes {self.dim} coordinate arrays, got "
                             f"{len(pts)}")
        trg = None
        if self.type == 3:
            trg = tuple(v for v in (s, t, u) if v is not None)
            if len(trg) != self.dim:
                raise ValueError(f"a {self.dim}D type-3 plan takes {self.dim} target arrays, "
                                 f"got {len(trg)}")
        self._plan = self._kind.build(self.dim, pts, trg, self.n_modes, self._opts, self.isign)
        self._adjoint = None
        self._points, self._targets = pts, trg

    def _apply(self, kind, plan, data, inner, out, what):
        rank = kind.rank(self.dim)
        n, single = _vectors(data, rank, inner=inner)
        if n != self.n_trans:
            raise ValueError(f"{what} got {n} vectors; the plan was made for "
                             f"n_trans={self.n_trans}")
        res = kind.run(plan, _stack_view(data, rank), n)
        return _deliver(res, single and self.n_trans == 1, self.dtype, out)

    def execute(self, data, out=None):
        if self._plan is None:
            raise RuntimeError("call setpts() before execute()")
        inner = self._kind.inner(self._plan, self.n_modes)
        return self._apply(self._kind, self._plan, data, inner, out, "execute")

    def execute_adjoint(self, data, out=None):
        """The adjoint of the planned transform: the sibling transform with
        the opposite sign (type 1 <-> type 2 at the same points; type 3 with
        sources and targets exchanged)."""
        if self._plan is None:
            raise RuntimeError("call setpts() before execute_adjoint()")
        adj = _KINDS[self._kind.adjoint_code]
        if self._adjoint is None:
            if self.type == 3:
                self._adjoint = adj.build(self.dim, self._targets, self._points, None,
                                          self._opts, -self.isign)
            else:
                self._adjoint = adj.build(self.dim, self._points, None, self.n_modes,
                                          self._opts, -self.isign)
        # the adjoint consumes what execute produces
        if self.type == 1:
            inner = tuple(self.n_modes)
        elif self.type == 2:
            inner = (self._plan.P,)
        else:
            inner = (self._plan.M,)
        return self._apply(adj, self._adjoint, data, inner, out, "execute_adjoint")
