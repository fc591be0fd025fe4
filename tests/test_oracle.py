"""Pins the CPU oracle (oracle/) before it is trusted as the checker.

Every check compares the oracle with something independent of it:
closed-form known answers, scipy's adaptive quadrature, numpy's own np.mod
/ ceil / stable argsort, numpy's FFT on equispaced points, and brute-force
Python loops on tiny inputs. A dropped term, a wrong sign or a transposed
index in the oracle fails at least one of them.
"""

import itertools

import numpy as np
import pytest
import scipy.integrate

TWO_PI = 2.0 * np.pi


# ------------------------------------------------------------------ sizing --

def _smooth235_table(limit):
    """All 2^a 3^b 5^c <= limit (generated, not tested by trial division)."""
    out = set()
    p2 = 1
    while p2 <= limit:
        p3 = p2
        while p3 <= limit:
            p5 = p3
            while p5 <= limit:
                out.add(p5)
                p5 *= 5
            p3 *= 3
        p2 *= 2
    return np.array(sorted(out))


def test_next235even_against_generated_table(oracle):
    tab = _smooth235_table(200_000)
    even = tab[tab % 2 == 0]
    for n in list(range(0, 3000)) + [4095, 4097, 8191, 10007, 65537, 99991, 123457]:
        exp = int(even[np.searchsorted(even, max(n, 2))])
        assert oracle.next235even(n) == exp, n


@pytest.mark.parametrize("eps,sigma,w,beta", [
    (1e-1, 2.0, 2, 4.4), (1e-2, 2.0, 3, 6.78), (1e-3, 2.0, 4, 9.52), (1e-4, 2.0, 5, 11.5),
    (1e-5, 2.0, 6, 13.8), (1e-6, 2.0, 7, 16.1), (1e-9, 2.0, 10, 23.0), (1e-15, 2.0, 16, 36.8),
    (1e-20, 2.0, 16, 36.8), (1e-5, 1.25, 9, 16.45566231965758),
])
def test_kernel_params_known_answers(oracle, eps, sigma, w, beta):
    """Known answers: w=6, beta=13.8 at eps 1e-5; w=7, beta=16.1 at 1e-6;
    sigma=1.25, eps 1e-5 -> w=9, beta = 0.97*pi*0.6*9."""
    ww, bb = oracle.kernel_params(eps, sigma)
    assert ww == w and abs(bb - beta) < 1e-9 * beta


def test_grid_sizes_known_answers(oracle):
    assert oracle.type12_grid((256, 256, 256), 1e-5)[2] == [512, 512, 512]
    assert oracle.type12_grid((1024, 1024), 1e-6)[2] == [2048, 2048]
    assert oracle.type12_grid((4096,), 1e-6)[2] == [8192]
    assert oracle.type12_grid((5,), 1e-6)[2] == [16]          # 2w = 14 floor, 235-smooth 16
    # type-3 cfg: sources in [-1,1] (X=1), targets in [-200,200] (S=200)
    nf, h, gam = oracle.set_nhg_type3(200.0, 1.0, 1.25, 9)
    assert (nf, round(gam, 12)) == (180, 0.36)
    assert abs(h - TWO_PI / 180) < 1e-15
    assert oracle.next235even(int(np.ceil(1.25 * nf))) == 240
    # degenerate extents (the 1D/2D type-3 embedding)
    assert oracle.set_nhg_type3(0.0, 0.0, 1.25, 9)[0] == 18


@pytest.mark.filterwarnings("ignore::scipy.integrate.IntegrationWarning")
@pytest.mark.parametrize("w,sigma", [(6, 2.0), (7, 2.0), (9, 1.25), (2, 2.0), (16, 2.0)])
def test_kernel_ft_against_adaptive_quadrature(oracle, w, sigma):
    """phihat(xi) = int psi(d) cos(xi d) dd. The 128-point Gauss-Legendre rule
    has its own error from the sqrt endpoint behaviour (measured <= 2e-8
    relative, at w = 2); a slip in the formula (a lost factor 2, the half
    width, the node map) is an O(1) error, so 1e-7 separates the two."""
    _, beta = oracle.kernel_params(10.0 ** -(w - 1) if sigma == 2.0 else 1e-5, sigma)
    xi = np.array([0.0, 0.3, 1.0, 1.7, np.pi / 2, 2.5, np.pi])
    got = oracle.kernel_ft(xi, beta, w)
    for k, x in enumerate(xi):
        f = lambda d, x=x: np.exp(beta * (np.sqrt(max(0.0, 1.0 - (2 * d / w) ** 2)) - 1.0)) * np.cos(x * d)
        ref, _ = scipy.integrate.quad(f, -w / 2, w / 2, limit=400, epsabs=1e-15, epsrel=1e-13)
        assert abs(got[k] - ref) <= 1e-7 * abs(ref), (w, x, got[k], ref)


# ----------------------------------------------------------------- setpts --

def _coords(rng, P):
    edge = np.array([0.0, -0.0, TWO_PI, -TWO_PI, np.pi, -np.pi, 1e-300, -1e-300, -5e-324,
                     -1e-17, 7e15, -7e15, 3 * TWO_PI, np.nextafter(TWO_PI, 0)])
    return np.concatenate([rng.uniform(-np.pi, np.pi, P), rng.uniform(-1e4, 1e4, P),
                           rng.standard_normal(P) * 1e-9, edge])


@pytest.mark.parametrize("prec64", [True, False])
@pytest.mark.parametrize("n,w", [(512, 6), (8192, 7), (180, 9), (14, 7), (37 * 2, 2)])
def test_setpts_matches_numpy_ops(oracle, prec64, n, w):
    """The C restatement reproduces numpy's own np.mod / division / ceil /
    astype sequence bit for bit (the reference's host path)."""
    rng = np.random.default_rng(3)
    x = _coords(rng, 20_000)
    i1, fr = oracle.setpts_t12([x], [n], w, prec64)
    rdt = np.float64 if prec64 else np.float32
    h = 2.0 * np.pi / n
    xi = np.mod(x, 2.0 * np.pi).astype(rdt) / rdt(h)
    ii = np.ceil(xi - rdt(w / 2.0)).astype(np.int32)
    ff = (xi - ii.astype(rdt)).astype(np.float32)
    assert np.array_equal(i1[0], ii)
    assert np.array_equal(fr[0].view(np.int32), ff.view(np.int32))


def test_setpts_invariants(oracle):
    rng = np.random.default_rng(4)
    x = [rng.uniform(-50, 50, 100_000) for _ in range(3)]
    n, w = [512, 480, 90], 6
    i1, fr = oracle.setpts_t12(x, n, w)
    for d in range(3):
        assert np.all(fr[d] > w / 2 - 1 - 1e-6) and np.all(fr[d] <= w / 2 + 1e-6)
        r = np.remainder(x[d], TWO_PI)
        assert np.allclose(i1[d] + fr[d].astype(np.float64), r / (TWO_PI / n[d]), atol=1e-6)


# ------------------------------------------------------------------- sort --

def test_stable_sort_equals_numpy_stable_argsort(oracle):
    rng = np.random.default_rng(5)
    for nk, P in [(1, 10), (17, 5000), (4096, 300_000), (1 << 20, 100_000)]:
        key = rng.integers(0, nk, P).astype(np.uint32)
        perm = oracle.stable_sort(key, nk)
        assert np.array_equal(perm, np.argsort(key, kind="stable").astype(np.uint32))
    with pytest.raises(ValueError):
        oracle.stable_sort(np.array([3], np.uint32), 3)


def test_bin_keys_definition(oracle):
    """key = row-major bin index of ((i1 + w//2) mod n) // m."""
    i1 = np.array([[-3, 0, 508, 511], [5, -2, 100, 47]], np.int32)
    key, nb = oracle.bin_keys(i1, [512, 48], [16, 12], 6)
    exp = [((a + 3) % 512 // 16) * 4 + ((b + 3) % 48 // 12) for a, b in zip(i1[0], i1[1])]
    assert nb == 32 * 4
    assert list(key) == exp


# ---------------------------------------------------------- direct sums --

def test_direct_sums_equal_fft_on_equispaced_points(oracle):
    """On x_j = 2 pi j / n the type-1/2 sums are DFTs."""
    rng = np.random.default_rng(6)
    n = 24
    g = np.arange(n) * TWO_PI / n
    X, Y = np.meshgrid(g, g, indexing="ij")
    c = rng.standard_normal((n, n)) + 1j * rng.standard_normal((n, n))
    k = np.arange(-(n // 2), n - n // 2)
    for isign in (+1, -1):
        f = oracle.dft_t1([X.ravel(), Y.ravel()], c.ravel(), [k, k], isign)
        F = np.fft.ifft2(c) * n * n if isign > 0 else np.fft.fft2(c)
        ref = F[np.ix_(k % n, k % n)]
        assert np.allclose(f, ref, atol=1e-9 * np.abs(ref).max())
        fk = rng.standard_normal((n, n)) + 1j * rng.standard_normal((n, n))
        c2 = oracle.dft_t2([X.ravel(), Y.ravel()], fk, isign)
        full = np.zeros((n, n), complex)
        full[np.ix_(k % n, k % n)] = fk
        G = np.fft.ifft2(full) * n * n if isign > 0 else np.fft.fft2(full)
        assert np.allclose(c2, G.ravel(), atol=1e-9 * np.abs(G).max())


def test_direct_t3_brute_force(oracle):
    rng = np.random.default_rng(7)
    x = [rng.uniform(-2, 2, 50) for _ in range(3)]
    s = [rng.uniform(-9, 9, 20) for _ in range(3)]
    c = rng.standard_normal(50) + 1j * rng.standard_normal(50)
    for isign in (+1, -1):
        got = oracle.dft_t3(x, c, s, isign)
        ref = np.array([sum(c[j] * np.exp(1j * isign * sum(s[d][k] * x[d][j] for d in range(3)))
                            for j in range(50)) for k in range(20)])
        assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_spread_brute_force(oracle):
    """The fp64 spread against a plain loop over taps on a tiny 2D grid."""
    rng = np.random.default_rng(8)
    n, w, beta = [16, 14], 5, 11.5
    x = [rng.uniform(-np.pi, np.pi, 7) for _ in range(2)]
    c = rng.standard_normal(7) + 1j * rng.standard_normal(7)
    i1, fr = oracle.setpts_t12(x, n, w)
    got = oracle.spread(i1, fr, c, n, w, beta)
    ref = np.zeros(n, complex)
    psi = lambda d: np.exp(beta * (np.sqrt(1 - (2 * d / w) ** 2) - 1)) if abs(d) <= w / 2 else 0.0
    for j in range(7):
        for a, b in itertools.product(range(w), range(w)):
            ref[(i1[0][j] + a) % n[0], (i1[1][j] + b) % n[1]] += \
                c[j] * psi(a - float(fr[0][j])) * psi(b - float(fr[1][j]))
    assert np.allclose(got, ref, rtol=1e-13, atol=1e-13)
    # interp is the adjoint of spread: <spread c, g> == <c, interp g>
    g = rng.standard_normal(n) + 1j * rng.standard_normal(n)
    lhs = np.vdot(g.ravel(), got.ravel())
    rhs = np.vdot(oracle.interp(i1, fr, g.conj(), w, beta).conj(), c)
    assert abs(lhs - rhs) < 1e-12 * abs(lhs)


# -------------------------------------------------------------- pipelines --

@pytest.mark.parametrize("dim,N", [(1, (87,)), (2, (48, 36)), (3, (21, 18, 14))])
@pytest.mark.parametrize("eps", [1e-3, 1e-6])
def test_pipelines_against_direct_sums(oracle, dim, N, eps):
    rng = np.random.default_rng(9)
    M = 3000
    x = [rng.uniform(-np.pi, np.pi, M) for _ in range(dim)]
    c = rng.standard_normal(M) + 1j * rng.standard_normal(M)
    ks = [np.arange(-(n // 2), n - n // 2) for n in N]
    for isign in (+1, -1):
        f = oracle.nufft_t1(x, c, N, eps, isign)
        assert oracle.rel_l2(f, oracle.dft_t1(x, c, ks, isign)) < 3 * eps
        fk = rng.standard_normal(N) + 1j * rng.standard_normal(N)
        c2 = oracle.nufft_t2(x, fk, eps, isign)
        assert oracle.rel_l2(c2, oracle.dft_t2(x, fk, isign)) < 3 * eps


@pytest.mark.parametrize("eps", [1e-3, 1e-4, 1e-5, 1e-6])
@pytest.mark.parametrize("centred", [True, False])
def test_type3_pipeline_against_direct_sum(oracle, eps, centred):
    """At sigma = 1.25 the ES kernel of the reference's sizing reaches a few
    eps (the same restatement's type-1 at sigma = 1.25 measures 1-2.5 eps),
    and type 3 passes through two such kernels, so the gate is 10 eps. Off-
    centre sources and targets (C, D != 0) exercise the pre/post phases: a
    wrong sign or a dropped centre there is an O(1) error."""
    rng = np.random.default_rng(10)
    xo, so = (0.0, 0.0) if centred else (2.5, 50.0)
    x = [xo + rng.uniform(-1, 1, 2000) for _ in range(3)]
    s = [so * (d + 1) + rng.uniform(-40, 40, 300) for d in range(3)]
    c = rng.standard_normal(2000) + 1j * rng.standard_normal(2000)
    for isign in (+1, -1):
        fe = oracle.dft_t3(x, c, s, isign)
        assert oracle.rel_l2(oracle.nufft_t3(x, c, s, eps, isign), fe) < 10 * eps
        if eps >= 1e-4:
            f32 = oracle.nufft_t3(x, c, s, eps, isign, spread64=False)
            assert oracle.rel_l2(f32, fe) < 10 * eps


def test_cpu_baseline_port_accuracy(oracle):
    rng = np.random.default_rng(11)
    M, N = 20_000, (20, 16, 12)
    x = [rng.uniform(-np.pi, np.pi, M) for _ in range(3)]
    c = (rng.standard_normal(M) + 1j * rng.standard_normal(M)).astype(np.complex64)
    f, t = oracle.cpu_type1_f32(x, c, N, 1e-5, workers=2)
    ks = [np.arange(-(n // 2), n - n // 2) for n in N]
    assert oracle.rel_l2(f, oracle.dft_t1(x, c, ks, +1)) < 1e-4
    assert t["total"] > 0


@pytest.mark.parametrize("prec", ["crit64", "coords64", "phases64", "fp32"])
def test_type3_setup_modes(oracle, prec):
    """t3_setup in each precision mode against what the mathematics fixes:
    - the cells and fractions rebuild the coordinate: the source at
      C + gam h (i1 + fr - nf/2), the target theta = h2 (i1 + fr - n_up/2),
      with fr in (w/2 - 1, w/2], to the rounding of the mode's rescale
      dtype (an off-by-one cell, a dropped centre or scale fails this);
    - pre = exp(i isign D.x) and post = exp(i isign C.(s - D)) / prod
      phihat(theta), evaluated here in fp64 with numpy's dot (another
      summation order), agree to the rounding of the mode's phase dtype;
    - a mode whose rescale (or phase) dtype is fp32 does round: its
      fractions (angles) differ from the fp64 mode's somewhere.
    The crit64 mode is also pinned end to end through nufft_t3 above."""
    rng = np.random.default_rng(12)
    x = [2.5 + rng.uniform(-1, 1, 3000) for _ in range(3)]
    s = [40.0 * (d + 1) + rng.uniform(-60, 60, 2000) for d in range(3)]
    for isign in (+1, -1):
        st = oracle.t3_setup(x, s, 1e-5, isign, 1.25, prec)
        ref = oracle.t3_setup(x, s, 1e-5, isign, 1.25, "crit64")
        w = st["w"]
        r32 = prec in ("fp32", "phases64")
        p32 = prec in ("fp32", "coords64")
        tol_r = 4e-7 if r32 else 1e-14
        for d in range(3):
            fr, i1 = st["fr"][d].astype(np.float64), st["i1"][d]
            assert fr.min() > w / 2 - 1 - 1e-5 and fr.max() <= w / 2 + 1e-5
            xr = st["C"][d] + st["gam"][d] * st["h"][d] * (i1 + fr - st["nf"][d] / 2)
            scale = st["gam"][d] * st["h"][d] * st["nf"][d]
            assert np.abs(xr - x[d]).max() <= (tol_r + 1.2e-7 * w) * scale
            tf, ti = st["t_fr"][d].astype(np.float64), st["t_i1"][d]
            assert tf.min() > w / 2 - 1 - 1e-5 and tf.max() <= w / 2 + 1e-5
            h2 = 2 * np.pi / st["n_up"][d]
            th = h2 * (ti + tf - st["n_up"][d] / 2)
            assert np.abs(th - st["theta"][d]).max() <= (tol_r + 1.2e-7 * w) * h2 * st["n_up"][d]
            th_exact = (s[d] - st["D"][d]) * (st["h"][d] * st["gam"][d])
            assert np.abs(st["theta"][d] - th_exact).max() <= tol_r * np.pi * 2
        X = np.stack(x)
        S = np.stack(s)
        ang_pre = np.asarray(st["D"]) @ X
        ang_post = np.asarray(st["C"]) @ (S - np.asarray(st["D"])[:, None])
        tol_p = 2e-7 * np.abs(ang_pre).max() if p32 else 1e-12
        assert np.abs(st["pre"] - np.exp(1j * isign * ang_pre)).max() <= tol_p
        tdec = np.prod([oracle.kernel_ft(th, st["beta"], w) for th in st["theta"]], axis=0)
        post = np.exp(1j * isign * ang_post) / tdec
        tol_q = 2e-7 * np.abs(ang_post).max() if p32 else 1e-12
        assert np.abs(st["post"] * tdec - post * tdec).max() <= tol_q
        if r32:
            assert not np.array_equal(st["fr"], ref["fr"])
        if p32:
            assert not np.array_equal(st["pre"], ref["pre"])


def test_f32_weight_emulation_modes(oracle):
    """The oracle's fp32 ES-weight emulations, used to locate the type-3
    error at eps 1e-6: on a 3D spread at sigma 1.25 (beta 16.5 and 18.3) the
    plain fp32 exponent beta (sqrt(1 - z^2) - 1) is off the fp64 grid by
    about beta x 3e-8 (the square root's rounding, multiplied by beta where
    the exponent cancels), while -beta z^2 / (1 + sqrt(1 - z^2)) in fp32 is
    off by about one fp32 rounding. A dropped term or a wrong sign in either
    form would move its grid far outside these bands."""
    for eps in (1e-5, 1e-6):
        w, beta = oracle.kernel_params(eps, 1.25)
        rng = np.random.default_rng(3)
        P, n = 4000, (48, 40, 36)
        x = [rng.uniform(-np.pi, np.pi, P) for _ in range(3)]
        c = rng.standard_normal(P) + 1j * rng.standard_normal(P)
        i1, fr = oracle.setpts_t12(x, n, w)
        g64 = oracle.spread(i1, fr, c, n, w, beta)
        e_plain = oracle.rel_l2(oracle.spread(i1, fr, c, n, w, beta, weights_f32="f32"), g64)
        e_stable = oracle.rel_l2(
            oracle.spread(i1, fr, c, n, w, beta, weights_f32="f32-stable"), g64)
        assert 2e-7 < e_plain < 2e-6, (eps, e_plain)
        assert 1e-8 < e_stable < 2e-7, (eps, e_stable)
        assert e_stable < e_plain / 4
        # the default restores fp64 weights
        assert oracle.rel_l2(oracle.spread(i1, fr, c, n, w, beta), g64) == 0.0
