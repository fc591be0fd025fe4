"""GPU checks of the owner-computes 2D y-sweep spread.

* point words (key: 64-column block of the first tap, y, reach bit; the
  in-block x cell above it), sorted fractions, perm and the key start table
  bit-exact against a numpy restatement;
* the spread grid against the oracle's fp64 spread on the same (i1, fr) for
  w = 2..8, clustered points (many batches per y), footprints wrapping in
  x and y on the smallest eligible grid (two blocks), and a y extent that is
  not a multiple of the segment;
* batched vectors == looped, and y-sweep == LDS-tile spread;
* 2D type-1 transforms through the y-sweep against the direct sum.
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _words_numpy(i1, n, w):
    """The y-sweep point word: key (bx*n1 + y)*2 + reach in bits 0-25, the
    in-block x cell of the first tap in bits 26-31."""
    x, y = (i1[d].astype(np.int64) % n[d] for d in range(2))
    lx = x % 64
    reach = (lx + w - 1 >= 64).astype(np.int64)
    key = ((x // 64) * n[1] + y) * 2 + reach
    word = key | (lx << 26)
    return key.astype(np.uint32), word.astype(np.uint32), (n[0] // 64) * n[1] * 2


@pytest.mark.parametrize("N,eps", [((64, 40), 1e-5), ((256, 100), 1e-3), ((96, 64), 1e-7)])
def test_ysweep_words_sort_and_starts(N, eps, oracle, mn):
    print(f"case ysweep words N={N} eps={eps}", flush=True)
    rng = np.random.default_rng(31)
    M = 50_000
    x = [rng.uniform(-np.pi, np.pi, M) for _ in range(2)]
    x[0][:4] = [-np.pi, np.pi, 0.0, -1e-300]   # fold edges
    p = mn.Type1PlanND(tuple(x), N, eps=eps)
    assert p.pts.kind == "ysweep"
    i1o, fro = oracle.setpts_t12(x, p.n_up, p.w)
    key, word, K = _words_numpy(i1o, p.n_up, p.w)
    ref = np.argsort(key, kind="stable")
    assert np.array_equal(p.pts.perm.cpu().numpy().view(np.uint32), ref.astype(np.uint32))
    assert np.array_equal(p.pts.word.cpu().numpy().view(np.uint32), word[ref])
    assert np.array_equal(p.pts.frs.cpu().numpy().view(np.int32), fro[:, ref].view(np.int32))
    ys = p.pts.ystart.cpu().numpy().astype(np.int64)
    assert np.array_equal(ys, np.searchsorted(key[ref], np.arange(K + 1), side="left"))


def _grid_check(oracle, mn, x, c, N, eps, tol=1e-5):
    from mlx_nufft_amd import _engine as E

    p = mn.Type1PlanND(tuple(x), N, eps=eps)
    assert p.pts.kind == "ysweep"
    grid = torch.empty(p.n_up, dtype=torch.complex64, device="cuda")
    E.spread_ysweep(p.pts, p.beta, torch.from_numpy(c).cuda(), grid)
    i1o, fro = oracle.setpts_t12(x, p.n_up, p.w)
    go = oracle.spread(i1o, fro, c, p.n_up, p.w, p.beta)
    err = oracle.rel_l2(grid.cpu().numpy(), go)
    assert err < tol, err
    return p


@pytest.mark.parametrize("eps", [1e-1, 1e-2, 1e-3, 1e-4, 1e-5, 1e-6, 1e-7])
def test_ysweep_widths(eps, oracle, mn):
    """w = 2 .. 8 through eps (sigma = 2)."""
    print(f"case ysweep width eps={eps}", flush=True)
    rng = np.random.default_rng(32)
    M = 40_000
    x = [rng.uniform(-np.pi, np.pi, M) for _ in range(2)]
    c = (rng.standard_normal(M) + 1j * rng.standard_normal(M)).astype(np.complex64)
    _grid_check(oracle, mn, x, c, (64, 50), eps)


def test_ysweep_clustered_and_wrapping(oracle, mn):
    """Points clustered at the periodic corner of a 128 x 40 grid (two
    blocks: the -x neighbour of block 0 is block 1, wrapping), many batches
    per y, footprints wrapping in x and y."""
    print("case ysweep clustered", flush=True)
    rng = np.random.default_rng(33)
    M = 60_000
    x = [np.concatenate([-np.pi + rng.uniform(0, 0.15, M // 2),
                         np.pi - rng.uniform(0, 0.15, M - M // 2)]) for _ in range(2)]
    c = (rng.standard_normal(M) + 1j * rng.standard_normal(M)).astype(np.complex64)
    p = _grid_check(oracle, mn, x, c, (64, 20), 1e-5)
    assert p.n_up[0] == 128


def test_ysweep_partial_segment(oracle, mn):
    """A y extent (n1 = 300) that is not a multiple of the segment."""
    print("case ysweep partial segment", flush=True)
    rng = np.random.default_rng(34)
    M = 60_000
    x = [rng.uniform(-np.pi, np.pi, M) for _ in range(2)]
    c = (rng.standard_normal(M) + 1j * rng.standard_normal(M)).astype(np.complex64)
    p = _grid_check(oracle, mn, x, c, (128, 150), 1e-5)
    assert p.n_up[1] % 32 != 0


def test_ysweep_batched_and_matches_tiles(mn, monkeypatch):
    """B vectors in one launch == one at a time (bit for bit), and the
    y-sweep grid == the LDS-tile spread grid."""
    from mlx_nufft_amd import _engine as E

    print("case ysweep batched + vs tiles", flush=True)
    rng = np.random.default_rng(35)
    M, B, N = 300_000, 3, (256, 200)
    x = [rng.uniform(-np.pi, np.pi, M) for _ in range(2)]
    cs = torch.from_numpy((rng.standard_normal((B, M)) + 1j * rng.standard_normal((B, M)))
                          .astype(np.complex64)).cuda()
    py = mn.Type1PlanND(tuple(x), N, eps=1e-6)
    assert py.pts.kind == "ysweep"
    gb = torch.empty((B, *py.n_up), dtype=torch.complex64, device="cuda")
    E.spread_ysweep(py.pts, py.beta, cs, gb)
    for b in range(B):
        g1 = torch.empty(py.n_up, dtype=torch.complex64, device="cuda")
        E.spread_ysweep(py.pts, py.beta, cs[b], g1)
        assert torch.equal(g1, gb[b])
    monkeypatch.setenv("MN_SPREAD", "tiles")
    pt = mn.Type1PlanND(tuple(x), N, eps=1e-6)
    assert pt.pts.kind == "tiles"
    gt = torch.empty(pt.n_up, dtype=torch.complex64, device="cuda")
    E.spread(pt.pts, pt.beta, cs[1], gt)
    assert float((gb[1] - gt).abs().norm() / gt.abs().norm()) < 1e-6


@pytest.mark.parametrize("N", [(64, 40), (128, 33)])
@pytest.mark.parametrize("isign", [+1, -1])
def test_type1_2d_ysweep_vs_direct(N, isign, oracle, mn):
    print(f"case ysweep t1 N={N} isign={isign}", flush=True)
    rng = np.random.default_rng(36)
    M, eps = 40_000, 1e-5
    x = [rng.uniform(-np.pi, np.pi, M) for _ in range(2)]
    c = (rng.standard_normal(M) + 1j * rng.standard_normal(M)).astype(np.complex64)
    p = mn.Type1PlanND(tuple(x), N, eps=eps, isign=isign)
    assert p.pts.kind == "ysweep"
    f = p.execute(c)
    modes = [np.arange(-(n // 2), n - n // 2) for n in N]
    fe = oracle.dft_t1(x, c, modes, isign)
    ref_err = oracle.rel_l2(oracle.nufft_t1(x, c, N, eps, isign), fe)
    err = oracle.rel_l2(f, fe)
    print(f"  err={err:.3e} ref_err={ref_err:.3e}")
    assert err <= max(eps, 2 * ref_err)
