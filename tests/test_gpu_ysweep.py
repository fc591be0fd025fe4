"""GPU checks of the two owner-computes 2D spreads: the VALU y-sweep
(kind "ysweep", forced with MN_SPREAD=ysweep) and the y-window MFMA sweep
(kind "ymfma", the default where its geometry applies).

* point words (y-sweep key: 64-column block of the first tap, y, reach
  bit, the in-block x cell above it; MFMA-sweep key: 16-column block,
  8-cell y-chunk, reach bit, the x and y cells in block and chunk above
  it), sorted fractions, perm and the key start table bit-exact against
  numpy restatements;
* the spread grid against the oracle's fp64 spread on the same (i1, fr) for
  w = 2..8, clustered points (many batches per y), footprints wrapping in
  x and y on the smallest eligible grids, and a y extent that is not a
  multiple of the segment;
* batched vectors == looped, and each sweep == LDS-tile spread;
* 2D type-1 transforms through each sweep against the direct sum.

Tolerance: the MFMA sweep's split fp16 products carry each term to about
2^-22, the same rel_l2 < 1e-5 gate against the fp64 oracle as the VALU
sweep, and 1e-6 against the fp32 tile spread.
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(params=["ysweep", "ymfma"])
def path(request, monkeypatch):
    """The 2D sweep under test: MN_SPREAD=ysweep forces the VALU y-sweep;
    without it eligible grids take the MFMA sweep."""
    if request.param == "ysweep":
        monkeypatch.setenv("MN_SPREAD", "ysweep")
    else:
        monkeypatch.delenv("MN_SPREAD", raising=False)
    return request.param


def _spread(E, p, c, grid):
    fn = E.spread_ymfma if p.pts.kind == "ymfma" else E.spread_ysweep
    fn(p.pts, p.beta, c, grid)


def _words_numpy(i1, n, w):
    """The y-sweep point word: key (bx*n1 + y)*2 + reach in bits 0-25, the
    in-block x cell of the first tap in bits 26-31."""
    x, y = (i1[d].astype(np.int64) % n[d] for d in range(2))
    lx = x % 64
    reach = (lx + w - 1 >= 64).astype(np.int64)
    key = ((x // 64) * n[1] + y) * 2 + reach
    word = key | (lx << 26)
    return key.astype(np.uint32), word.astype(np.uint32), (n[0] // 64) * n[1] * 2


def _ym_words_numpy(i1, n, w):
    """The MFMA-sweep point word: key ((x//16)*(n1/8) + y//8)*2 + reach in
    bits 0-24, x mod 16 in bits 25-28, y mod 8 in bits 29-31."""
    x, y = (i1[d].astype(np.int64) % n[d] for d in range(2))
    lx, ly, nyc = x % 16, y % 8, n[1] // 8
    reach = (lx + w - 1 >= 16).astype(np.int64)
    key = ((x // 16) * nyc + y // 8) * 2 + reach
    word = key | (lx << 25) | (ly << 29)
    return key.astype(np.uint32), word.astype(np.uint32), (n[0] // 16) * nyc * 2


@pytest.mark.parametrize("N,eps", [((64, 40), 1e-5), ((256, 100), 1e-3), ((96, 64), 1e-7)])
def test_ysweep_words_sort_and_starts(N, eps, path, oracle, mn):
    print(f"case {path} words N={N} eps={eps}", flush=True)
    rng = np.random.default_rng(31)
    M = 50_000
    x = [rng.uniform(-np.pi, np.pi, M) for _ in range(2)]
    x[0][:4] = [-np.pi, np.pi, 0.0, -1e-300]   # fold edges
    p = mn.Type1PlanND(tuple(x), N, eps=eps)
    assert p.pts.kind == path
    i1o, fro = oracle.setpts_t12(x, p.n_up, p.w)
    key, word, K = (_words_numpy if path == "ysweep" else _ym_words_numpy)(i1o, p.n_up, p.w)
    ref = np.argsort(key, kind="stable")
    assert np.array_equal(p.pts.perm.cpu().numpy().view(np.uint32), ref.astype(np.uint32))
    assert np.array_equal(p.pts.word.cpu().numpy().view(np.uint32), word[ref])
    assert np.array_equal(p.pts.frs.cpu().numpy().view(np.int32), fro[:, ref].view(np.int32))
    ys = p.pts.ystart.cpu().numpy().astype(np.int64)
    assert np.array_equal(ys, np.searchsorted(key[ref], np.arange(K + 1), side="left"))


def _grid_check(oracle, mn, x, c, N, eps, path, tol=1e-5):
    from mlx_nufft_amd import _engine as E

    p = mn.Type1PlanND(tuple(x), N, eps=eps)
    assert p.pts.kind == path
    grid = torch.empty(p.n_up, dtype=torch.complex64, device="cuda")
    _spread(E, p, torch.from_numpy(c).cuda(), grid)
    i1o, fro = oracle.setpts_t12(x, p.n_up, p.w)
    go = oracle.spread(i1o, fro, c, p.n_up, p.w, p.beta)
    err = oracle.rel_l2(grid.cpu().numpy(), go)
    assert err < tol, err
    return p


@pytest.mark.parametrize("eps", [1e-1, 1e-2, 1e-3, 1e-4, 1e-5, 1e-6, 1e-7])
def test_ysweep_widths(eps, path, oracle, mn):
    """w = 2 .. 8 through eps (sigma = 2)."""
    print(f"case {path} width eps={eps}", flush=True)
    rng = np.random.default_rng(32)
    M = 40_000
    x = [rng.uniform(-np.pi, np.pi, M) for _ in range(2)]
    c = (rng.standard_normal(M) + 1j * rng.standard_normal(M)).astype(np.complex64)
    _grid_check(oracle, mn, x, c, (64, 48), eps, path)


def test_ysweep_clustered_and_wrapping(path, oracle, mn):
    """Points clustered at the periodic corner of a 128 x 40 grid (y-sweep:
    two blocks, the -x neighbour of block 0 is block 1, wrapping), many
    batches per y, footprints wrapping in x and y."""
    print(f"case {path} clustered", flush=True)
    rng = np.random.default_rng(33)
    M = 60_000
    x = [np.concatenate([-np.pi + rng.uniform(0, 0.15, M // 2),
                         np.pi - rng.uniform(0, 0.15, M - M // 2)]) for _ in range(2)]
    c = (rng.standard_normal(M) + 1j * rng.standard_normal(M)).astype(np.complex64)
    p = _grid_check(oracle, mn, x, c, (64, 20), 1e-5, path)
    assert p.n_up[0] == 128


def test_ymfma_smallest_grid(oracle, mn, monkeypatch):
    """The smallest MFMA-sweep grid, 32 x 16 (two blocks, two y-chunks, so
    each chunk's window wraps onto the other), with clustered and spread
    points at w = 7 and w = 2."""
    monkeypatch.delenv("MN_SPREAD", raising=False)
    rng = np.random.default_rng(37)
    for eps, M in ((1e-6, 30_000), (1e-1, 20_000)):
        print(f"case ymfma smallest eps={eps}", flush=True)
        x = [np.concatenate([-np.pi + rng.uniform(0, 0.5, M // 2),
                             rng.uniform(-np.pi, np.pi, M - M // 2)]) for _ in range(2)]
        c = (rng.standard_normal(M) + 1j * rng.standard_normal(M)).astype(np.complex64)
        p = _grid_check(oracle, mn, x, c, (16, 8), eps, "ymfma")
        assert tuple(p.n_up) == (32, 16)


def test_ysweep_partial_segment(path, oracle, mn):
    """A y extent (n1 = 200) that is not a multiple of the segment."""
    print(f"case {path} partial segment", flush=True)
    rng = np.random.default_rng(34)
    M = 60_000
    x = [rng.uniform(-np.pi, np.pi, M) for _ in range(2)]
    c = (rng.standard_normal(M) + 1j * rng.standard_normal(M)).astype(np.complex64)
    p = _grid_check(oracle, mn, x, c, (128, 100), 1e-5, path)
    assert p.n_up[1] % 32 != 0


@pytest.mark.parametrize("B", [3, 8, 11])
def test_ysweep_batched_and_matches_tiles(B, path, mn, monkeypatch):
    """B vectors in one launch == one at a time (bit for bit; B = 11 runs a
    full group of 8 and a partial one), and the sweep's grid == the
    LDS-tile spread grid."""
    from mlx_nufft_amd import _engine as E

    print(f"case {path} batched B={B} + vs tiles", flush=True)
    rng = np.random.default_rng(35)
    M, N = 300_000, (256, 200)
    x = [rng.uniform(-np.pi, np.pi, M) for _ in range(2)]
    cs = torch.from_numpy((rng.standard_normal((B, M)) + 1j * rng.standard_normal((B, M)))
                          .astype(np.complex64)).cuda()
    py = mn.Type1PlanND(tuple(x), N, eps=1e-6)
    assert py.pts.kind == path
    gb = torch.empty((B, *py.n_up), dtype=torch.complex64, device="cuda")
    _spread(E, py, cs, gb)
    for b in range(B):
        g1 = torch.empty(py.n_up, dtype=torch.complex64, device="cuda")
        _spread(E, py, cs[b], g1)
        assert torch.equal(g1, gb[b])
    monkeypatch.setenv("MN_SPREAD", "tiles")
    pt = mn.Type1PlanND(tuple(x), N, eps=1e-6)
    assert pt.pts.kind == "tiles"
    gt = torch.empty(pt.n_up, dtype=torch.complex64, device="cuda")
    E.spread(pt.pts, pt.beta, cs[1], gt)
    assert float((gb[1] - gt).abs().norm() / gt.abs().norm()) < 1e-6


@pytest.mark.parametrize("N", [(64, 40), (128, 33), (96, 45)])
@pytest.mark.parametrize("isign", [+1, -1])
def test_type1_2d_ysweep_vs_direct(N, isign, path, oracle, mn):
    print(f"case {path} t1 N={N} isign={isign}", flush=True)
    rng = np.random.default_rng(36)
    M, eps = 40_000, 1e-5
    x = [rng.uniform(-np.pi, np.pi, M) for _ in range(2)]
    c = (rng.standard_normal(M) + 1j * rng.standard_normal(M)).astype(np.complex64)
    p = mn.Type1PlanND(tuple(x), N, eps=eps, isign=isign)
    # n_up (192, 90) takes the VALU y-sweep on both paths (90 is not a
    # multiple of 8)
    assert p.pts.kind == (path if p.n_up[1] % 8 == 0 else "ysweep")
    f = p.execute(c)
    modes = [np.arange(-(n // 2), n - n // 2) for n in N]
    fe = oracle.dft_t1(x, c, modes, isign)
    ref_err = oracle.rel_l2(oracle.nufft_t1(x, c, N, eps, isign), fe)
    err = oracle.rel_l2(f, fe)
    print(f"  err={err:.3e} ref_err={ref_err:.3e}")
    assert err <= max(eps, 2 * ref_err)


@pytest.mark.parametrize("B", [1, 2, 3, 4, 5, 8, 9])
def test_pointmajor_transpose(B, mn):
    """mn_pointmajor_c64 (vector-major strengths to the point-major layout
    the y-window MFMA sweep reads) equals torch's transpose bit for bit,
    for the LDS-tiled B = 2, 4, 8 and the per-element other B, with P not a
    multiple of any tile (partial last tiles)."""
    from mlx_nufft_amd import _lib as L

    print(f"case pointmajor B={B}", flush=True)
    rng = np.random.default_rng(60 + B)
    for P in (1, 1000, 2048 * 3 + 17):
        cs = torch.from_numpy((rng.standard_normal((B, P)) + 1j * rng.standard_normal((B, P)))
                              .astype(np.complex64)).cuda()
        out = torch.full((P, B), float("nan"), dtype=torch.complex64, device="cuda")
        L.check(L.lib().mn_pointmajor_c64(B, P, L.ptr(cs), L.ptr(out), L.stream()), "pointmajor")
        assert torch.equal(out, cs.t().contiguous()), (B, P)
