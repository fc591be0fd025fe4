"""Z-gather interpolation (3D type-2 over the z-sweep point state, through
mn_interp_zgather) against the oracle's fp64 interp and the staged-tile
interp, with the batch, scale and zero-grid properties of its fp16 hi/lo
operands.

Tolerance: the hi/lo split carries each grid value and y-weight to about
2^-22 and accumulates in f32, so the interpolated values agree with the
fp64 oracle to rel_l2 < 2e-6 and with the fp32 tile interp to 3e-6 of the
largest value (both differ from the oracle by about 1e-6).
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

# (mode box, eps -> w, clustered at the periodic corner, points): fine grids
# 64x48x40 (w 7), 16^3 (the smallest, w 7), 80x72x150 (w 4, a partial last
# z-chunk), 48^3 (w 2), 64x40x30 (w 8, a partial last z-chunk), 32x32x64 (w 6),
# 32x32x12 (w 6: two z-chunks, the second partial, so the 16-slot ring holds
# every z cell more than once), 32x48x12 (w 3)
CASES = [((32, 24, 20), 1e-6, False, 30_000), ((8, 8, 8), 1e-6, True, 20_000),
         ((40, 36, 75), 1e-3, False, 200_000), ((24, 24, 24), 1e-1, False, 120_000),
         ((32, 20, 13), 1e-7, True, 60_000), ((16, 16, 32), 1e-5, False, 50_000),
         ((16, 16, 4), 1e-5, True, 40_000), ((16, 24, 6), 1e-2, False, 30_000)]


def _pts(rng, M, cluster):
    if cluster:
        return [np.concatenate([-np.pi + rng.uniform(0, 0.3, M // 2),
                                np.pi - rng.uniform(0, 0.3, M - M // 2)]) for _ in range(3)]
    return [rng.uniform(-np.pi, np.pi, M) for _ in range(3)]


def _cplx(rng, shape):
    return (rng.standard_normal(shape) + 1j * rng.standard_normal(shape)).astype(np.complex64)


def _zgather(E, p, g, B=1):
    out = torch.empty((B, p.P), dtype=torch.complex64, device="cuda")
    E.interp_zgather(p.pts, p.beta, g, out, B=B)
    return out


@pytest.mark.parametrize("N,eps,cluster,M", CASES)
def test_zgather_vs_oracle_and_tiles(N, eps, cluster, M, oracle, mn, monkeypatch):
    from mlx_nufft_amd import _engine as E

    print(f"case zgather N={N} eps={eps} cluster={cluster} M={M}", flush=True)
    rng = np.random.default_rng(61)
    x = _pts(rng, M, cluster)
    p = mn.Type2PlanND(tuple(x), N, eps=eps)
    assert p.pts.kind == "zgather", "the case must select the z-gather"
    g = _cplx(rng, tuple(p.n_up))
    gd = torch.from_numpy(g).cuda()
    oz = _zgather(E, p, gd)[0]
    i1o, fro = oracle.setpts_t12(x, p.n_up, p.w)
    oo = oracle.interp(i1o, fro, g, p.w, p.beta)
    err = oracle.rel_l2(oz.cpu().numpy(), oo)
    monkeypatch.setenv("MN_INTERP", "tiles")
    pt = mn.Type2PlanND(tuple(x), N, eps=eps)
    assert pt.pts.kind not in ("zsweep", "zgather")
    ot = torch.empty(M, dtype=torch.complex64, device="cuda")
    E.interp(pt.pts, pt.beta, gd, ot)
    dt = float((oz - ot).abs().max() / ot.abs().max())
    print(f"  w={p.w} n_up={p.n_up} rel_l2 vs oracle {err:.3e}, max vs tiles {dt:.3e}")
    assert err < 2e-6
    assert dt < 3e-6


def test_zgather_batch_and_segments(mn):
    """B grids in one launch equal B single launches bit for bit, and the
    z-segment length (one or several per wave column) does not change a bit."""
    from mlx_nufft_amd import _engine as E

    print("case zgather batch", flush=True)
    rng = np.random.default_rng(62)
    M, N = 80_000, (24, 32, 40)
    p = mn.Type2PlanND(tuple(_pts(rng, M, False)), N, eps=1e-5)
    assert p.pts.kind == "zgather"
    gs = torch.from_numpy(_cplx(rng, (3, *p.n_up))).cuda()
    ob = _zgather(E, p, gs, B=3)
    for b in range(3):
        o1 = _zgather(E, p, gs[b])[0]
        assert torch.equal(ob[b], o1)
    for zseg in (8, 24, 80):
        oz = torch.empty((1, M), dtype=torch.complex64, device="cuda")
        E.interp_zgather(p.pts, p.beta, gs[0], oz, zseg=zseg)
        assert torch.equal(oz[0], ob[0])


def test_zgather_scale_and_zero(mn):
    """Power-of-two scalings of the grid scale the result exactly (the
    per-half fp16 scales follow the grid), and a zero grid gives zeros."""
    from mlx_nufft_amd import _engine as E

    print("case zgather scale", flush=True)
    rng = np.random.default_rng(63)
    M, N = 40_000, (16, 16, 16)
    p = mn.Type2PlanND(tuple(_pts(rng, M, False)), N, eps=1e-5)
    assert p.pts.kind == "zgather"
    g = torch.from_numpy(_cplx(rng, tuple(p.n_up))).cuda()
    o = _zgather(E, p, g)[0]
    for k in (-100, 100):
        os_ = _zgather(E, p, g * 2.0 ** k)[0]
        assert torch.equal(os_, o * 2.0 ** k), k
    oz = _zgather(E, p, torch.zeros_like(g))[0]
    assert torch.count_nonzero(oz) == 0
