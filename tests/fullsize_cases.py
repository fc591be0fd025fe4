"""Inputs of the BASELINE.json configurations at their full sizes, built from
fixed seeds so that the fixture generator (tests/golden/make_fullsize_ref.py,
run on the CPU) and the GPU tests (tests/test_gpu_fullsize.py) see the same
bits. Each case also fixes the sample -- modes for type 1, points for
type 2, targets for type 3 -- on which the exact direct sum is evaluated.

The shapes and distributions are the configurations' own (BASELINE.json
configs[0..4]); numpy default_rng seeds 0 (data) and 100 (samples).
"""

import numpy as np

PI = np.pi


def _cplx(rng, shape):
    return (rng.standard_normal(shape) + 1j * rng.standard_normal(shape)).astype(np.complex64)


def _mode_sample(N, per_dim):
    """per_dim distinct modes per axis (sorted), drawn from the modeord-0 box."""
    rng = np.random.default_rng(100)
    return [np.sort(rng.choice(np.arange(-(n // 2), n - n // 2), per_dim, replace=False))
            for n in N]


def _mode_sample_edges(N, per_dim):
    """per_dim distinct modes per axis (sorted): both ends of the modeord-0
    box, -(n // 2) and n - n // 2 - 1, plus per_dim - 2 drawn from between."""
    rng = np.random.default_rng(100)
    out = []
    for n in N:
        lo, hi = -(n // 2), n - n // 2 - 1
        mid = rng.choice(np.arange(lo + 1, hi), per_dim - 2, replace=False)
        out.append(np.sort(np.concatenate([[lo, hi], mid])))
    return out


def _point_sample(P, count):
    rng = np.random.default_rng(100)
    return np.sort(rng.choice(P, count, replace=False))


def cfg0_1d_t1():
    """1D type-1: M = 1e5, N = 4096, eps 1e-6, isign +1 (all modes sampled)."""
    rng = np.random.default_rng(0)
    M = 100_000
    x = [rng.uniform(-PI, PI, M)]
    c = _cplx(rng, M)
    N = (4096,)
    return {"x": x, "c": c, "N": N, "eps": 1e-6, "isign": +1,
            "modes": [np.arange(-(N[0] // 2), N[0] - N[0] // 2)]}


def cfg1_2d_t1_batched():
    """2D type-1, 8 strength vectors sharing M = 1e7 points, N = 1024^2,
    eps 1e-6, isign +1; an 8 x 8 sub-grid of modes is sampled."""
    rng = np.random.default_rng(0)
    M = 10_000_000
    x = [rng.uniform(-PI, PI, M) for _ in range(2)]
    cs = _cplx(rng, (8, M))
    N = (1024, 1024)
    return {"x": x, "cs": cs, "N": N, "eps": 1e-6, "isign": +1, "modes": _mode_sample(N, 8),
            "checked": (0, 7)}


def cfg2_2d_t2_radial():
    """2D type-2 on 512 spokes x 2048 radial samples (angles uniform in
    [0, pi), radii evenly spaced in [-pi, pi)), f of 1024^2 modes, eps 1e-6,
    isign -1; 1024 points are sampled."""
    rng = np.random.default_rng(0)
    f = _cplx(rng, (1024, 1024))
    theta = rng.uniform(0.0, PI, 512)
    r = np.linspace(-PI, PI, 2048, endpoint=False)
    x = [np.outer(np.cos(theta), r).ravel(), np.outer(np.sin(theta), r).ravel()]
    return {"x": x, "f": f, "eps": 1e-6, "isign": -1,
            "points": _point_sample(x[0].size, 1024)}


def cfg3_3d_t1():
    """3D type-1: M = 2e7, N = 256^3, eps 1e-5, isign +1; an 8 x 8 x 8
    sub-grid of modes, including both ends of every axis, is sampled (the
    type-2 round trip samples 512 points)."""
    rng = np.random.default_rng(0)
    M = 20_000_000
    x = [rng.uniform(-PI, PI, M) for _ in range(3)]
    c = _cplx(rng, M)
    N = (256, 256, 256)
    return {"x": x, "c": c, "N": N, "eps": 1e-5, "isign": +1,
            "modes": _mode_sample_edges(N, 8), "points": _point_sample(M, 512)}


def cfg4_3d_t3():
    """3D type-3: 1e6 sources uniform in [-1, 1]^3, 1e6 targets uniform in
    [-200, 200]^3, eps 1e-5, isign +1; 256 targets are sampled. Also expi on
    1e7 phases uniform in [-1e6, 1e6]."""
    rng = np.random.default_rng(0)
    n = 1_000_000
    x = [rng.uniform(-1.0, 1.0, n) for _ in range(3)]
    s = [rng.uniform(-200.0, 200.0, n) for _ in range(3)]
    c = _cplx(rng, n)
    return {"x": x, "s": s, "c": c, "eps": 1e-5, "isign": +1,
            "targets": _point_sample(n, 256)}


def expi_phases():
    rng = np.random.default_rng(0)
    return rng.uniform(-1e6, 1e6, 10_000_000)
