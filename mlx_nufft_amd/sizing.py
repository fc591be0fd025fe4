"""Plan-time sizing: fine-grid sizes, ES kernel width/shape, kernel Fourier
transform and type-3 grid parameters (host fp64 scalars and small vectors).

These follow the FINUFFT-family formulas the reference uses
(ref: mlx_nufft/sizing.py:13-111), so grid sizes and kernel shapes match.
"""

import numpy as np

PI = np.pi


def next235even(n: int) -> int:
    """Smallest even integer >= max(n, 2) with no prime factor above 5.

    ref: sizing.py:13-25.
    """
    n = max(int(n), 2)
    n += n & 1
    while True:
        r = n
        for p in (2, 3, 5):
            while r % p == 0:
                r //= p
        if r == 1:
            return n
        n += 2


def kernel_params(eps: float, upsampfac: float):
    """(w, beta) of the ES kernel for tolerance eps at upsampling factor sigma.

    sigma == 2: w = ceil(log10(10/eps)); otherwise
    w = ceil(-ln(eps) / (pi*sqrt(1 - 1/sigma))); w is clipped to [2, 16].
    beta = (beta/w)*w with beta/w = 2.20, 2.26, 2.38 for w = 2, 3, 4 and 2.30
    above (sigma == 2), or 0.97*pi*(1 - 1/(2 sigma)) otherwise.
    ref: sizing.py:28-50.
    """
    if upsampfac == 2.0:
        w = int(np.ceil(-np.log10(eps / 10.0)))
    else:
        w = int(np.ceil(-np.log(eps) / (PI * np.sqrt(1.0 - 1.0 / upsampfac))))
    w = min(max(w, 2), 16)
    ratio = {2: 2.20, 3: 2.26, 4: 2.38}.get(w, 2.30)
    if upsampfac != 2.0:
        ratio = 0.97 * PI * (1.0 - 1.0 / (2.0 * upsampfac))
    return w, ratio * w


def inner_kernel_params(eps: float, sigma_inner: float):
    """Width/beta of the type-3 inner interpolation kernel at sigma_inner.

    ref: gpu_t3.py:279-284.
    """
    w = int(np.ceil(-np.log(eps) / (PI * np.sqrt(1.0 - 1.0 / sigma_inner))))
    w = min(max(w, 2), 16)
    return w, 0.97 * PI * (1.0 - 1.0 / (2.0 * sigma_inner)) * w


def es_kernel(d, beta, w):
    """psi(d) = exp(beta*(sqrt(1 - (2d/w)^2) - 1)) for |d| <= w/2, else 0.

    ref: sizing.py:53-62.
    """
    z2 = (2.0 * np.asarray(d, dtype=np.float64) / w) ** 2
    out = np.zeros_like(z2)
    m = z2 <= 1.0
    out[m] = np.exp(beta * (np.sqrt(1.0 - z2[m]) - 1.0))
    return out


_GL = {}


def quadrature(beta, w, nquad=128):
    """Nodes dq on [0, w/2] and weights fq = GL weight * psi(dq) such that
    phihat(xi) = 2 * sum_q fq[q] cos(xi dq[q]) (even kernel).

    ref: sizing.py:74-85 (128-point Gauss-Legendre on [0, w/2]).
    """
    if nquad not in _GL:
        _GL[nquad] = np.polynomial.legendre.leggauss(nquad)
    t, wt = _GL[nquad]
    dq = 0.5 * (t + 1.0) * (w / 2.0)
    fq = wt * (w / 4.0) * es_kernel(dq, beta, w)
    return dq, fq


def kernel_ft(xi, beta, w, nquad=128):
    """phihat(xi) = int_{-w/2}^{w/2} psi(d) e^{i xi d} dd (real, even), fp64.

    ref: sizing.py:74-85.
    """
    xi = np.atleast_1d(np.asarray(xi, dtype=np.float64))
    dq, fq = quadrature(beta, w, nquad)
    return 2.0 * (fq @ np.cos(np.outer(dq, xi)))


def set_nhg_type3(S, X, upsampfac, w):
    """Type-3 fine-grid size nf, spacing h = 2pi/nf and scale gamma for one
    dim, from the target half-width S and source half-width X.

    ref: sizing.py:88-111.
    """
    Xs, Ss = X, S
    if X == 0.0:
        if S == 0.0:
            Xs, Ss = 1.0, 1.0
        else:
            Xs = max(Xs, 1.0 / S)
    else:
        Ss = max(Ss, 1.0 / X)
    nf = int(2.0 * upsampfac * Ss * Xs / PI + (w + 1))
    nf = next235even(max(nf, 2 * w))
    return nf, 2.0 * PI / nf, nf / (2.0 * upsampfac * Ss)
