"""The legacy 3D plans with their default arguments, and the spread_method
choices of the ND plans, against exact direct sums.

- Type1Plan/Type2Plan (ref: mlx_nufft/types12.py:159-186): eps 1e-5,
  upsampfac 1.25, isign +1 for both, called with defaults only. A plan
  that used the opposite sign would land far from the direct sum.
- spread_method "auto", "od" and "gm" (ref: nd.py:397-404, 869-874): each
  choice that applies must reach the same accuracy; "gm" must select the
  LDS-tile spread (type 1) or the direct gather (3D type 2).

Gate: max(eps, 2 ref_err), ref_err being the CPU fp64 oracle's error at the
same w, beta and fine grid.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _modes(N):
    return [np.arange(-(n // 2), n - n // 2) for n in N]


def _gate(oracle, label, got, exact, approx, eps):
    err = oracle.rel_l2(got, exact)
    gate = max(eps, 2.0 * oracle.rel_l2(approx, exact))
    print(f"  {label}: err={err:.3e} gate={gate:.3e}", flush=True)
    assert err <= gate, label
    return err


def test_legacy_plans_default_arguments(oracle, mn):
    print("case legacy Type1Plan/Type2Plan defaults", flush=True)
    rng = np.random.default_rng(31)
    P, N, eps = 5000, (16, 12, 10), 1e-5
    x = [rng.uniform(-np.pi, np.pi, P) for _ in range(3)]
    c = rng.standard_normal(P) + 1j * rng.standard_normal(P)

    f = mn.Type1Plan(x, N).execute(c)
    assert f.shape == N
    exact = oracle.dft_t1(x, c, _modes(N), +1)
    _gate(oracle, "Type1Plan", f, exact, oracle.nufft_t1(x, c, N, eps, +1, upsampfac=1.25), eps)

    fk = rng.standard_normal(N) + 1j * rng.standard_normal(N)
    plan2 = mn.Type2Plan(x, N)
    assert plan2.isign == +1 and plan2.sigma == 1.25 and plan2.eps == 1e-5
    got = plan2.execute(fk)
    assert got.shape == (P,)
    exact2 = oracle.dft_t2(x, fk, +1)
    _gate(oracle, "Type2Plan", got, exact2, oracle.nufft_t2(x, fk, eps, +1, upsampfac=1.25), eps)
    # the conjugate-sign transform is a different result entirely
    assert oracle.rel_l2(got, oracle.dft_t2(x, fk, -1)) > 0.5
    # results come back in caller order whether or not the plan sorts
    got_sorted = mn.Type2Plan(x, N, sort_points=True).execute(fk)
    assert oracle.rel_l2(got_sorted, got) < 1e-6


@pytest.mark.parametrize("dim,N", [(3, (32, 24, 20)), (2, (64, 48)), (1, (1100,))])
def test_spread_methods(dim, N, oracle, mn):
    from mlx_nufft_amd.nd import od_applicable

    print(f"case spread_method dim={dim} N={N}", flush=True)
    rng = np.random.default_rng(32 + dim)
    P, eps = 24000, 1e-5
    x = [rng.uniform(-np.pi, np.pi, P) for _ in range(dim)]
    c = rng.standard_normal(P) + 1j * rng.standard_normal(P)
    fk = rng.standard_normal(N) + 1j * rng.standard_normal(N)
    exact1 = oracle.dft_t1(x, c, _modes(N), +1)
    exact2 = oracle.dft_t2(x, fk, -1)
    approx1 = oracle.nufft_t1(x, c, N, eps, +1)
    approx2 = oracle.nufft_t2(x, fk, eps, -1)
    res1, res2 = {}, {}
    for m in ("auto", "od", "gm"):
        p1 = mn.Type1PlanND(x, N, eps=eps, isign=+1, spread_method=m)
        if m == "od":
            assert od_applicable(dim, p1.w, p1.n_up, P), "the case must let od apply"
        res1[m] = _gate(oracle, f"t1 {m} ({p1.pts.kind})", p1.execute(c), exact1, approx1, eps)
        if m == "gm":
            assert p1.pts.kind == "tiles"
        p2 = mn.Type2PlanND(x, N, eps=eps, isign=-1, spread_method=m)
        res2[m] = _gate(oracle, f"t2 {m}", p2.execute(fk), exact2, approx2, eps)
        if m == "gm":
            assert p2._gather_direct() == (dim == 3)
