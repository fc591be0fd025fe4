"""CPU oracle of the MI355X NUFFT engine -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the checker (or as the reported CPU baseline). The
product package mlx_nufft_amd never imports it.

It restates the reference's algorithm on the CPU (numpy + the C library
oracle/liboracle.so built from oracle/nufft_oracle.c):
  * sizing: next235even, kernel_params, es_kernel, kernel_ft,
    set_nhg_type3                              (ref: mlx_nufft/sizing.py)
  * setpts / bin keys / stable sort            (ref: nd.py:152-165, 308-314)
  * fp64 type-1 / type-2 pipelines at the engine's w, beta, n_up
                                               (ref: nd.py:386-1119)
  * fp64 type-3 pipeline                       (ref: ref_t3.py:48-221)
  * exact fp64 direct sums (OpenMP C)          (ref: harness/gen.py:93-114)
  * rel_l2                                     (ref: harness/gen.py:117-120)
  * the CPU baseline: fp32 OpenMP spread + scipy.fft (a port of the same
    algorithm; finufft itself is not installed here).

How each piece is pinned (tests/test_oracle.py): sizing against closed-form
known answers, numpy's Gauss-Legendre and scipy's adaptive quadrature;
setpts against numpy's own np.mod/ceil on random and edge inputs plus the
fr range invariant; the sort against numpy's stable argsort; every
pipeline against the exact direct sums (and those against numpy's FFT on
uniform points and brute-force loops on tiny inputs).
"""

import ctypes
import os
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
PI = np.pi

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        vp = ctypes.c_void_p
        i64 = ctypes.c_int64
        L.or_setpts_t12.argtypes = [ctypes.c_int, i64, vp, vp, ctypes.c_int, ctypes.c_int, vp, vp]
        L.or_bin_keys.argtypes = [ctypes.c_int, i64, vp, vp, vp, vp, ctypes.c_int, vp]
        L.or_stable_sort.argtypes = [i64, vp, i64, vp]
        L.or_stable_sort.restype = ctypes.c_int
        L.or_spread.argtypes = [ctypes.c_int, i64, vp, vp, vp, vp, ctypes.c_int, ctypes.c_double, vp]
        L.or_interp.argtypes = [ctypes.c_int, i64, vp, vp, vp, vp, ctypes.c_int, ctypes.c_double, vp]
        L.or_spread_f32.argtypes = [ctypes.c_int, i64, vp, vp, vp, vp, ctypes.c_int, ctypes.c_double,
                                    i64, vp]
        L.or_spread_f32.restype = ctypes.c_int
        L.or_dft_t1.argtypes = [ctypes.c_int, i64, vp, vp, vp, vp, ctypes.c_int, vp]
        L.or_dft_t2.argtypes = [ctypes.c_int, vp, vp, vp, ctypes.c_int, i64, vp, vp]
        L.or_dft_t3.argtypes = [i64, vp, vp, vp, ctypes.c_int, i64, vp, vp]
        L.or_set_weights_f32.argtypes = [ctypes.c_int]
        _lib = L
    return _lib


def _pa(arrs):
    """Array of pointers (keeps the numpy arrays alive in the caller)."""
    return (ctypes.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])


def _p(a):
    return ctypes.c_void_p(a.ctypes.data)


# --------------------------------------------------------------- sizing ----

def next235even(n):
    """ref: sizing.py:13-25."""
    n = max(int(n), 2)
    if n % 2:
        n += 1
    while True:
        m = n
        for p in (2, 3, 5):
            while m % p == 0:
                m //= p
        if m == 1:
            return n
        n += 2


def kernel_params(eps, upsampfac):
    """ref: sizing.py:28-50."""
    if upsampfac == 2.0:
        ns = int(np.ceil(-np.log10(eps / 10.0)))
    else:
        ns = int(np.ceil(-np.log(eps) / (PI * np.sqrt(1.0 - 1.0 / upsampfac))))
    ns = max(2, min(ns, 16))
    r = 2.30
    if ns == 2:
        r = 2.20
    elif ns == 3:
        r = 2.26
    elif ns == 4:
        r = 2.38
    if upsampfac != 2.0:
        r = 0.97 * PI * (1.0 - 1.0 / (2.0 * upsampfac))
    return ns, r * ns


def es_kernel(d, beta, w):
    """ref: sizing.py:53-62."""
    z2 = (2.0 * np.asarray(d, dtype=np.float64) / w) ** 2
    out = np.zeros_like(z2)
    m = z2 <= 1.0
    out[m] = np.exp(beta * (np.sqrt(1.0 - z2[m]) - 1.0))
    return out


def kernel_ft(xi, beta, w, nquad=128):
    """phihat(xi) by nquad-point Gauss-Legendre on [0, w/2] (ref: sizing.py:74-85)."""
    xi = np.atleast_1d(np.asarray(xi, dtype=np.float64))
    t, wt = np.polynomial.legendre.leggauss(nquad)
    d = 0.5 * (t + 1.0) * (w / 2.0)
    return 2.0 * ((wt * (w / 4.0)) * es_kernel(d, beta, w)) @ np.cos(np.outer(d, xi))


def set_nhg_type3(S, X, upsampfac, w):
    """ref: sizing.py:88-111."""
    Xs, Ss = X, S
    if X == 0.0:
        if S == 0.0:
            Xs, Ss = 1.0, 1.0
        else:
            Xs = max(Xs, 1.0 / S)
    else:
        Ss = max(Ss, 1.0 / X)
    nf = int(2.0 * upsampfac * Ss * Xs / PI + w + 1)
    if nf < 2 * w:
        nf = 2 * w
    nf = next235even(nf)
    return nf, 2.0 * PI / nf, nf / (2.0 * upsampfac * Ss)


def type12_grid(N, eps, upsampfac=2.0):
    """(w, beta, n_up) of a type-1/2 plan (ref: nd.py:122-125)."""
    w, beta = kernel_params(eps, upsampfac)
    n_up = [next235even(max(2 * w, int(np.ceil(upsampfac * n)))) for n in N]
    return w, beta, n_up


# ------------------------------------------------------- setpts / sort ----

def setpts_t12(x, n_up, w, prec64=True):
    """(i1 int32 [dim,P], fr float32 [dim,P]) in caller order."""
    x = [np.ascontiguousarray(np.asarray(v, dtype=np.float64).ravel()) for v in x]
    dim, P = len(x), x[0].size
    i1 = np.empty((dim, P), np.int32)
    fr = np.empty((dim, P), np.float32)
    n = np.asarray(list(n_up) + [1] * (3 - dim), np.int64)
    lib().or_setpts_t12(dim, P, _pa(x), _p(n), int(w), int(bool(prec64)),
                        _pa([i1[d] for d in range(dim)]), _pa([fr[d] for d in range(dim)]))
    return i1, fr


def bin_keys(i1, n_up, m, w):
    dim, P = i1.shape
    n = np.asarray(list(n_up) + [1] * (3 - dim), np.int64)
    mm = np.asarray(list(m) + [1] * (3 - dim), np.int32)
    nb = np.asarray([-(-int(a) // int(b)) for a, b in zip(n_up, m)] + [1] * (3 - dim), np.int32)
    key = np.empty(P, np.uint32)
    i1c = [np.ascontiguousarray(i1[d]) for d in range(dim)]
    lib().or_bin_keys(dim, P, _pa(i1c), _p(n), _p(mm), _p(nb), int(w), _p(key))
    return key, int(np.prod(nb[:dim]))


def stable_sort(key, nkeys):
    key = np.ascontiguousarray(key, dtype=np.uint32)
    perm = np.empty(key.size, np.uint32)
    if lib().or_stable_sort(key.size, _p(key), int(nkeys), _p(perm)) != 0:
        raise ValueError("stable_sort: key out of range")
    return perm


# --------------------------------------------------------- spread/interp ---

class _weights_f32:
    """Within the block the oracle's spread and interp evaluate the ES
    weights in fp32 (products and sums stay fp64): True or "f32" as the
    GPU's type-1/2 kernels do, "f32-stable" with the exponent rewritten
    without cancellation, as the GPU's type-3 spread does."""

    def __init__(self, mode):
        self.mode = {False: 0, True: 1, "f32": 1, "f32-stable": 2}[mode]

    def __enter__(self):
        lib().or_set_weights_f32(self.mode)

    def __exit__(self, *exc):
        lib().or_set_weights_f32(0)


def spread(i1, fr, c, n, w, beta, weights_f32=False):
    """fp64 spread onto the periodic grid n (complex128 array of shape n);
    weights_f32 evaluates the ES weights in fp32 (the GPU's formula)."""
    dim, P = i1.shape
    grid = np.zeros(tuple(n), np.complex128)
    cc = np.ascontiguousarray(np.asarray(c, dtype=np.complex128).ravel())
    nn = np.asarray(list(n) + [1] * (3 - dim), np.int64)
    i1c = [np.ascontiguousarray(i1[d]) for d in range(dim)]
    frc = [np.ascontiguousarray(fr[d]) for d in range(dim)]
    with _weights_f32(weights_f32):
        lib().or_spread(dim, P, _pa(i1c), _pa(frc), _p(cc), _p(nn), int(w), float(beta),
                        _p(grid))
    return grid


def interp(i1, fr, grid, w, beta, weights_f32=False):
    dim, P = i1.shape
    g = np.ascontiguousarray(grid, dtype=np.complex128)
    nn = np.asarray(list(g.shape) + [1] * (3 - dim), np.int64)
    out = np.empty(P, np.complex128)
    i1c = [np.ascontiguousarray(i1[d]) for d in range(dim)]
    frc = [np.ascontiguousarray(fr[d]) for d in range(dim)]
    with _weights_f32(weights_f32):
        lib().or_interp(dim, P, _pa(i1c), _pa(frc), _p(g), _p(nn), int(w), float(beta),
                        _p(out))
    return out


def _decs(N, n_up, beta, w):
    return [1.0 / kernel_ft(2.0 * PI * np.arange(-(Nd // 2), Nd - Nd // 2) / nd, beta, w)
            for Nd, nd in zip(N, n_up)]


def _outer(vecs):
    out = vecs[0]
    for v in vecs[1:]:
        out = np.multiply.outer(out, v)
    return out


def _fftn(H, isign):
    """Unnormalised DFT with e^{i isign ...}."""
    if isign > 0:
        return np.fft.ifftn(H) * H.size
    return np.fft.fftn(H)


def nufft_t1(x, c, N, eps, isign=+1, upsampfac=2.0):
    """fp64 CPU type-1 at the engine's (w, beta, n_up): f over the modeord=0 box."""
    w, beta, n_up = type12_grid(N, eps, upsampfac)
    i1, fr = setpts_t12(x, n_up, w)
    F = _fftn(spread(i1, fr, c, n_up, w, beta), isign)
    idx = np.ix_(*[np.arange(-(Nd // 2), Nd - Nd // 2) % nd for Nd, nd in zip(N, n_up)])
    return F[idx] * _outer(_decs(N, n_up, beta, w))


def nufft_t2(x, f, eps, isign=-1, upsampfac=2.0):
    """fp64 CPU type-2 at the engine's (w, beta, n_up)."""
    N = f.shape
    w, beta, n_up = type12_grid(N, eps, upsampfac)
    i1, fr = setpts_t12(x, n_up, w)
    H = np.zeros(n_up, np.complex128)
    idx = np.ix_(*[np.arange(-(Nd // 2), Nd - Nd // 2) % nd for Nd, nd in zip(N, n_up)])
    H[idx] = f * _outer(_decs(N, n_up, beta, w))
    return interp(i1, fr, _fftn(H, isign), w, beta)


def spread_f32(i1, fr, c, n, w, beta):
    """Spread with fp32 kernel evaluation and fp32 accumulation (the
    reference's spread64=False stage flag, ref_t3.py:168, 300-317)."""
    dim, P = i1.shape
    grid = np.empty(tuple(n), np.complex64)
    c32 = np.ascontiguousarray(np.asarray(c, np.complex64).ravel())
    nn = np.asarray(list(n) + [1] * (3 - dim), np.int64)
    i1c = [np.ascontiguousarray(i1[d]) for d in range(dim)]
    frc = [np.ascontiguousarray(fr[d]) for d in range(dim)]
    if lib().or_spread_f32(dim, P, _pa(i1c), _pa(frc), _p(c32), _p(nn), int(w), float(beta),
                           int(w), _p(grid)):
        raise MemoryError("or_spread_f32 failed")
    return grid.astype(np.complex128)


T3_PRECISIONS = ("fp32", "coords64", "phases64", "crit64")


def t3_setup(x, s, eps=1e-5, isign=+1, upsampfac=1.25, prec="crit64"):
    """Type-3 plan setup (3D) as the reference's host path computes it, in
    each precision mode: the sizing scalars (C, D, nf, h, gam, n_up;
    ref: gpu_t3.py:326-342), the targets' cells, fractions, theta and
    post factor (ref: gpu_t3.py:344-377) and the sources' cells, fractions
    and prephase (ref: gpu_t3.py:474-488). prec picks the dtype of the
    coordinate rescale (rdt: fp64 for crit64/coords64) and of the phase
    angles (pdt: fp64 for crit64/phases64); the operation order is the
    reference's, elementwise, so every fp32 step rounds where it does
    there. Returned arrays are in caller order."""
    if prec not in T3_PRECISIONS:
        raise ValueError(prec)
    rdt = np.float64 if prec in ("crit64", "coords64") else np.float32
    pdt = np.float64 if prec in ("crit64", "phases64") else np.float32
    w, beta = kernel_params(eps, upsampfac)
    isign = 1 if isign >= 0 else -1
    x = [np.asarray(v, np.float64).ravel() for v in x]
    s = [np.asarray(v, np.float64).ravel() for v in s]
    nf, h, gam, C, D = [], [], [], [], []
    for d in range(3):
        xlo, xhi = float(x[d].min()), float(x[d].max())
        slo, shi = s[d].min(), s[d].max()
        C.append(0.5 * (xlo + xhi))
        D.append(0.5 * (slo + shi))
        a, b, g = set_nhg_type3(0.5 * (shi - slo), 0.5 * (xhi - xlo), upsampfac, w)
        nf.append(a)
        h.append(b)
        gam.append(g)
    n_up = [next235even(int(np.ceil(upsampfac * n))) for n in nf]
    out = dict(w=w, beta=beta, nf=nf, h=h, gam=gam, C=C, D=D, n_up=n_up)

    ss = [v.astype(rdt) for v in s]
    t_i1 = np.empty((3, s[0].size), np.int32)
    t_fr = np.empty((3, s[0].size), np.float32)
    theta = []
    for d in range(3):
        hd = 2.0 * PI / nf[d]
        th = (ss[d] - rdt(D[d])) * rdt(hd * gam[d])
        theta.append(th.astype(np.float64))
        lam = th / rdt(2.0 * PI / n_up[d]) + rdt(n_up[d] / 2.0)
        t_i1[d] = np.ceil(lam - rdt(w / 2.0)).astype(np.int32)
        t_fr[d] = (lam - t_i1[d].astype(rdt)).astype(np.float32)
    sp = [v.astype(pdt) for v in s]
    post_ang = sum(pdt(C[d]) * (sp[d] - pdt(D[d])) for d in range(3))
    tdec = np.ones(s[0].size)
    for d in range(3):
        tdec *= kernel_ft(theta[d], beta, w)
    out.update(t_i1=t_i1, t_fr=t_fr, theta=theta, tdec=tdec,
               post=np.exp(1j * isign * post_ang.astype(np.float64)) / tdec)

    xs = [v.astype(rdt) for v in x]
    i1 = np.empty((3, x[0].size), np.int32)
    fr = np.empty((3, x[0].size), np.float32)
    for d in range(3):
        hd = 2.0 * PI / nf[d]
        xi = (xs[d] - rdt(C[d])) / rdt(gam[d]) / rdt(hd) + rdt(nf[d] / 2.0)
        i1[d] = np.ceil(xi - rdt(w / 2.0)).astype(np.int32)
        fr[d] = (xi - i1[d].astype(rdt)).astype(np.float32)
    xp = [v.astype(pdt) for v in x]
    pre_ang = sum(pdt(D[d]) * xp[d] for d in range(3))
    out.update(i1=i1, fr=fr, pre=np.exp(1j * isign * pre_ang.astype(np.float64)))
    return out


def nufft_t3(x, c, s, eps=1e-5, isign=+1, upsampfac=1.25, spread64=True,
             weights_f32=(False, False)):
    """CPU type-3 (3D), following ref_t3.py:48-221 with the crit64 setup of
    t3_setup: all stages fp64, or with the spread stage in fp32
    (spread64=False, the reference's most precision-sensitive fp32 stage,
    ref: harness/diagnose_ref.py:21-41). weights_f32 = (spread, interp)
    evaluates the ES weights of that fp64 stage in fp32 as the GPU does."""
    st = t3_setup(x, s, eps, isign, upsampfac, "crit64")
    w, beta, nf, n_up = st["w"], st["beta"], st["nf"], st["n_up"]
    cp = np.asarray(c, np.complex128) * st["pre"]
    if spread64:
        b = spread(st["i1"], st["fr"], cp, nf, w, beta, weights_f32=weights_f32[0])
    else:
        b = spread_f32(st["i1"], st["fr"], cp, nf, w, beta)
    decs = []
    for d in range(3):
        q = np.arange(-nf[d] // 2, nf[d] // 2, dtype=np.float64)
        decs.append(((-1.0) ** np.abs(q)) / kernel_ft(2.0 * PI * q / n_up[d], beta, w))
    H = np.zeros(n_up, np.complex128)
    H[np.ix_(*[np.arange(-nf[d] // 2, nf[d] // 2) % n_up[d] for d in range(3)])] = \
        b * _outer(decs)
    v = _fftn(H, isign)
    return interp(st["t_i1"], st["t_fr"], v, w, beta, weights_f32=weights_f32[1]) * st["post"]


# ----------------------------------------------------------- direct sums ---

def dft_t1(x, c, kvecs, isign=+1):
    """Exact f on the tensor grid of integer modes kvecs[0] x kvecs[1] x ..."""
    dim = len(x)
    x = [np.ascontiguousarray(np.asarray(v, np.float64).ravel()) for v in x]
    cc = np.ascontiguousarray(np.asarray(c, np.complex128).ravel())
    ks = [np.ascontiguousarray(np.asarray(k, np.int64)) for k in kvecs]
    nk = np.asarray([k.size for k in ks] + [1] * (3 - dim), np.int64)
    out = np.empty(tuple(k.size for k in ks), np.complex128)
    lib().or_dft_t1(dim, x[0].size, _pa(x), _p(cc), _p(nk), _pa(ks), int(isign), _p(out))
    return out


def dft_t2(x, f, isign=-1, idx=None):
    """Exact c_j at the points idx (all if None) for modes f (modeord=0)."""
    dim = len(x)
    x = [np.ascontiguousarray(np.asarray(v, np.float64).ravel()) for v in x]
    ff = np.ascontiguousarray(np.asarray(f, np.complex128))
    N = np.asarray(list(ff.shape) + [1] * (3 - dim), np.int64)
    idx = np.arange(x[0].size) if idx is None else np.asarray(idx)
    idx = np.ascontiguousarray(idx, dtype=np.int64)
    out = np.empty(idx.size, np.complex128)
    lib().or_dft_t2(dim, _pa(x), _p(ff), _p(N), int(isign), idx.size, _p(idx), _p(out))
    return out


def dft_t3(x, c, s, isign=+1, idx=None):
    """Exact f_k = sum_j c_j e^{i isign s_k.x_j} (3D) at targets idx."""
    x = [np.ascontiguousarray(np.asarray(v, np.float64).ravel()) for v in x]
    s = [np.ascontiguousarray(np.asarray(v, np.float64).ravel()) for v in s]
    cc = np.ascontiguousarray(np.asarray(c, np.complex128).ravel())
    idx = np.arange(s[0].size) if idx is None else np.asarray(idx)
    idx = np.ascontiguousarray(idx, dtype=np.int64)
    out = np.empty(idx.size, np.complex128)
    lib().or_dft_t3(x[0].size, _pa(x), _p(cc), _pa(s), int(isign), idx.size, _p(idx), _p(out))
    return out


def rel_l2(u, ref):
    """ref: harness/gen.py:117-120."""
    u = np.asarray(u).ravel()
    ref = np.asarray(ref).ravel()
    return float(np.linalg.norm(u - ref) / np.linalg.norm(ref))


# ---------------------------------------------------------- CPU baseline ---

def cpu_type1_f32(x, c, N, eps, isign=+1, workers=None, upsampfac=2.0):
    """CPU baseline: the same type-1 algorithm in fp32 with OpenMP spreading
    and scipy.fft (multithreaded) -- a port, not finufft. Returns (f, times)."""
    import time

    import scipy.fft

    workers = workers or os.cpu_count()
    t0 = time.perf_counter()
    w, beta, n_up = type12_grid(N, eps, upsampfac)
    i1, fr = setpts_t12(x, n_up, w)
    t1 = time.perf_counter()
    dim, P = i1.shape
    grid = np.empty(tuple(n_up), np.complex64)
    cc = np.ascontiguousarray(np.asarray(c, np.complex64).ravel())
    nn = np.asarray(list(n_up) + [1] * (3 - dim), np.int64)
    i1c = [np.ascontiguousarray(i1[d]) for d in range(dim)]
    frc = [np.ascontiguousarray(fr[d]) for d in range(dim)]
    rc = lib().or_spread_f32(dim, P, _pa(i1c), _pa(frc), _p(cc), _p(nn), int(w), float(beta),
                             max(int(w), n_up[0] // max(2, 2 * (workers or 1))), _p(grid))
    if rc:
        raise MemoryError("or_spread_f32 failed")
    t2 = time.perf_counter()
    if isign > 0:
        F = scipy.fft.ifftn(grid, workers=workers, norm="forward", overwrite_x=True)
    else:
        F = scipy.fft.fftn(grid, workers=workers, overwrite_x=True)
    t3 = time.perf_counter()
    idx = np.ix_(*[np.arange(-(Nd // 2), Nd - Nd // 2) % nd for Nd, nd in zip(N, n_up)])
    f = F[idx] * _outer([d.astype(np.float32) for d in _decs(N, n_up, beta, w)])
    t4 = time.perf_counter()
    return f, {"setpts": t1 - t0, "spread": t2 - t1, "fft": t3 - t2, "deconv": t4 - t3,
               "total": t4 - t0}
