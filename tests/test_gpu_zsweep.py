"""GPU checks of the owner-computes z-sweep spread.

* point words (key: block of the first tap, z, reach class in [00, 01, 11,
  10] order; in-block x/y cell above it), sorted fractions, perm and the key
  start table bit-exact against a numpy restatement;
* the spread grid against the oracle's fp64 spread on the same (i1, fr) for
  edge geometries: clustered points (more than 64 points per z-step of one
  block), 16-wide grids (the -x/-y neighbour block wraps), a z extent that
  is not a multiple of the segment, and w = 2..8;
* z-sweep == LDS-tile spread on the same plan inputs, with strengths read
  through perm or pre-permuted into sorted order.
"""

import numpy as np
import pytest
import torch
from zsweep_words import words_numpy as _words_numpy

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("N,eps", [((32, 24, 20), 1e-5), ((8, 8, 20), 1e-3), ((64, 64, 64), 1e-6)])
def test_zsweep_words_sort_and_starts(N, eps, oracle, mn):
    """Words, sorted fractions and perm bit-exact; zstart[k] = first sorted
    index with key >= k."""
    print(f"case zsweep words N={N} eps={eps}", flush=True)
    rng = np.random.default_rng(21)
    M = 50_000
    x = [rng.uniform(-np.pi, np.pi, M) for _ in range(3)]
    x[0][:4] = [-np.pi, np.pi, 0.0, -1e-300]   # fold edges
    p = mn.Type1PlanND(tuple(x), N, eps=eps)
    assert p.pts.kind == "zsweep"
    i1o, fro = oracle.setpts_t12(x, p.n_up, p.w)
    key, word, K = _words_numpy(i1o, p.n_up, p.w)
    ref = np.argsort(key, kind="stable")
    perm = p.pts.perm.cpu().numpy().view(np.uint32)
    assert np.array_equal(perm, ref.astype(np.uint32))
    assert np.array_equal(p.pts.word.cpu().numpy().view(np.uint32), word[ref])
    assert np.array_equal(p.pts.frs.cpu().numpy().view(np.int32), fro[:, ref].view(np.int32))
    zs = p.pts.zstart.cpu().numpy().astype(np.int64)
    exp = np.searchsorted(key[ref], np.arange(K + 1), side="left")
    assert np.array_equal(zs, exp)


def test_zsweep_starts_sparse(mn):
    """Few points far apart: long key gaps, filled by whole waves."""
    print("case zsweep sparse starts", flush=True)
    rng = np.random.default_rng(26)
    x = [rng.uniform(-np.pi, np.pi, 7) for _ in range(3)]
    p = mn.Type1PlanND(tuple(x), (64, 64, 64), eps=1e-5)
    key = p.pts.word.cpu().numpy().view(np.uint32) & ((1 << 23) - 1)
    zs = p.pts.zstart.cpu().numpy().astype(np.int64)
    assert np.array_equal(zs, np.searchsorted(key, np.arange(p.pts.K + 1), side="left"))


def _grid_check(oracle, mn, x, c, N, eps, tol=1e-5):
    from mlx_nufft_amd import _engine as E

    p = mn.Type1PlanND(tuple(x), N, eps=eps)
    assert p.pts.kind == "zsweep"
    grid = torch.empty(p.n_up, dtype=torch.complex64, device="cuda")
    E.spread_zsweep(p.pts, p.beta, torch.from_numpy(c).cuda(), grid)
    i1o, fro = oracle.setpts_t12(x, p.n_up, p.w)
    go = oracle.spread(i1o, fro, c, p.n_up, p.w, p.beta)
    err = oracle.rel_l2(grid.cpu().numpy(), go)
    assert err < tol, err
    return p


@pytest.mark.parametrize("eps", [1e-1, 1e-2, 1e-3, 1e-4, 1e-5, 1e-6, 1e-7])
def test_zsweep_widths(eps, oracle, mn):
    """w = 2 .. 8 through eps (sigma = 2)."""
    print(f"case zsweep width eps={eps}", flush=True)
    rng = np.random.default_rng(22)
    M = 20_000
    x = [rng.uniform(-np.pi, np.pi, M) for _ in range(3)]
    c = (rng.standard_normal(M) + 1j * rng.standard_normal(M)).astype(np.complex64)
    _grid_check(oracle, mn, x, c, (24, 20, 18), eps)


def test_zsweep_clustered_and_wrapping(oracle, mn):
    """Points clustered at the periodic corner (many per block and z, and
    footprints wrapping in x, y, z) on a 16x16 grid."""
    print("case zsweep clustered", flush=True)
    rng = np.random.default_rng(23)
    M = 40_000
    h = 2 * np.pi / 16
    x = [np.concatenate([-np.pi + rng.uniform(0, 3 * h, M // 2),
                         np.pi - rng.uniform(0, 3 * h, M - M // 2)]) for _ in range(3)]
    c = (rng.standard_normal(M) + 1j * rng.standard_normal(M)).astype(np.complex64)
    _grid_check(oracle, mn, x, c, (8, 8, 8), 1e-5)


def test_zsweep_partial_band(oracle, mn):
    """Workgroups go segment-major in bands of 16 block rows along x: a grid
    of more than 16 block rows that is not a multiple of 16 ends in a partial
    band, and three z-segments repeat the bands. Every cell must still be
    written exactly once."""
    print("case zsweep partial band", flush=True)
    rng = np.random.default_rng(27)
    M = 30_000
    x = [rng.uniform(-np.pi, np.pi, M) for _ in range(3)]
    c = (rng.standard_normal(M) + 1j * rng.standard_normal(M)).astype(np.complex64)
    p = _grid_check(oracle, mn, x, c, (76, 20, 150), 1e-5)
    nbx = p.n_up[0] // 8
    assert nbx > 16 and nbx % 16 != 0, p.n_up
    assert p.n_up[2] > 2 * 128, p.n_up


def test_zsweep_partial_segment(oracle, mn):
    """A z extent (n2 = 300) that is a multiple of neither the 128-cell
    segment nor the 8-cell chunk: the last chunk is partial, and the
    periodic chunk below z = 0 starts its slots 4 cells up."""
    print("case zsweep partial segment", flush=True)
    rng = np.random.default_rng(24)
    M = 60_000
    x = [rng.uniform(-np.pi, np.pi, M) for _ in range(3)]
    c = (rng.standard_normal(M) + 1j * rng.standard_normal(M)).astype(np.complex64)
    p = _grid_check(oracle, mn, x, c, (16, 16, 150), 1e-5)
    assert p.n_up[2] % 128 != 0 and p.n_up[2] % 8 != 0


def test_zsweep_matches_tiles(mn, monkeypatch):
    from mlx_nufft_amd import _engine as E

    print("case zsweep vs tiles", flush=True)
    rng = np.random.default_rng(25)
    M = 200_000
    x = [rng.uniform(-np.pi, np.pi, M) for _ in range(3)]
    c = torch.from_numpy((rng.standard_normal(M) + 1j * rng.standard_normal(M))
                         .astype(np.complex64)).cuda()
    pz = mn.Type1PlanND(tuple(x), (64, 64, 48), eps=1e-5)
    monkeypatch.setenv("MN_SPREAD", "tiles")
    pt = mn.Type1PlanND(tuple(x), (64, 64, 48), eps=1e-5)
    assert pz.pts.kind == "zsweep" and pt.pts.kind == "tiles"
    gz = torch.empty(pz.n_up, dtype=torch.complex64, device="cuda")
    gt = torch.empty(pt.n_up, dtype=torch.complex64, device="cuda")
    E.spread_zsweep(pz.pts, pz.beta, c, gz)
    E.spread(pt.pts, pt.beta, c, gt)
    assert float((gz - gt).abs().norm() / gt.abs().norm()) < 1e-6
    cs = torch.empty_like(c)
    E.permute_c64(pz.pts.perm, c, cs)
    assert torch.equal(cs, c[pz.pts.perm.long()])
    gp = torch.empty_like(gz)
    E.spread_zsweep(pz.pts, pz.beta, cs, gp, presorted=True)
    assert torch.equal(gp, gz)


def test_zsweep_matches_tiles_bench_grid(mn, monkeypatch):
    """The bench's grid (3D type-1, M = 2e7 uniform points, N = 256^3,
    eps 1e-5: a 512^3 fine grid, w = 6): the z-sweep's split-fp16 MFMA
    products against the tile spread's fp32 products accumulated in fp64,
    over the whole grid. Gate 1e-6 relative l2 (fp32 rounding of the weight
    products and of the stored grid is about 1e-7)."""
    from mlx_nufft_amd import _engine as E

    print("case zsweep vs tiles at 512^3, M=2e7", flush=True)
    rng = np.random.default_rng(0)
    M = 20_000_000
    x = tuple(torch.from_numpy(rng.uniform(-np.pi, np.pi, M)).cuda() for _ in range(3))
    c = torch.from_numpy((rng.standard_normal(M) + 1j * rng.standard_normal(M))
                         .astype(np.complex64)).cuda()
    pz = mn.Type1PlanND(x, (256, 256, 256), eps=1e-5)
    assert pz.pts.kind == "zsweep" and pz.w == 6 and list(pz.n_up) == [512] * 3
    gz = torch.empty(pz.n_up, dtype=torch.complex64, device="cuda")
    E.spread_zsweep(pz.pts, pz.beta, c, gz)
    del pz
    monkeypatch.setenv("MN_SPREAD", "tiles")
    pt = mn.Type1PlanND(x, (256, 256, 256), eps=1e-5)
    assert pt.pts.kind == "tiles"
    gt = torch.empty(pt.n_up, dtype=torch.complex64, device="cuda")
    E.spread(pt.pts, pt.beta, c, gt)
    rel = float((gz - gt).abs().norm() / gt.abs().norm())
    worst = float((gz - gt).abs().max() / gt.abs().max())
    print(f"  rel l2 {rel:.3e}, max |diff| / max |grid| {worst:.3e}")
    assert rel < 1e-6


@pytest.mark.parametrize("N,eps", [((64, 64, 48), 1e-5), ((32, 48, 40), 1e-7), ((48, 32, 64), 1e-2)])
def test_zsweep_segments(N, eps, oracle, mn):
    """Segments of 8, 16, 128 and 256 cells (8 and 16 put a segment edge in
    most footprints) spread the same points to the same grid within fp32
    rounding, every cell written (the grid starts as NaN), and the 128-cell
    grid matches the oracle."""
    from mlx_nufft_amd import _engine as E

    print(f"case zsweep segments N={N} eps={eps}", flush=True)
    rng = np.random.default_rng(27)
    M = 150_000
    x = [rng.uniform(-np.pi, np.pi, M) for _ in range(3)]
    c = (rng.standard_normal(M) + 1j * rng.standard_normal(M)).astype(np.complex64)
    cd = torch.from_numpy(c).cuda()
    p = mn.Type1PlanND(tuple(x), N, eps=eps)
    assert p.pts.kind == "zsweep"
    grids = {}
    for zseg in (8, 16, 128, 256):
        g = torch.full(p.n_up, float("nan"), dtype=torch.complex64, device="cuda")
        E.spread_zsweep(p.pts, p.beta, cd, g, zseg=zseg)
        assert bool(torch.isfinite(torch.view_as_real(g)).all()), zseg
        grids[zseg] = g
    ref = grids[128]
    for zseg, g in grids.items():
        rel = float((g - ref).abs().norm() / ref.abs().norm())
        print(f"  zseg {zseg}: rel diff {rel:.2e}")
        assert rel < 1e-6, zseg
    i1o, fro = oracle.setpts_t12(x, p.n_up, p.w)
    go = oracle.spread(i1o, fro, c, p.n_up, p.w, p.beta)
    assert oracle.rel_l2(ref.cpu().numpy(), go) < 1e-5


@pytest.mark.parametrize("case", ["tiny", "huge", "mixed", "sparse", "tiny36", "huge36"])
def test_zsweep_mfma_strength_range(case, oracle, mn):
    """The fp16 product path scales strengths per wave by a power of two
    (rescaling what it holds when a batch brings a larger one): strengths
    at 1e-30 and 1e30, at 1e-36 and 1e36 (near the ends of fp32's range), a
    mix where 1 % of the points are 1e8 times larger, and mostly-zero
    strengths (whole batches of zeros) all give the oracle's fp64 grid
    within 1e-5, with every cell finite."""
    from mlx_nufft_amd import _engine as E

    print(f"case zsweep strength range {case}", flush=True)
    rng = np.random.default_rng(28)
    M = 120_000
    x = [rng.uniform(-np.pi, np.pi, M) for _ in range(3)]
    c = rng.standard_normal(M) + 1j * rng.standard_normal(M)
    scale = {"tiny": 1e-30, "huge": 1e30, "tiny36": 1e-36, "huge36": 1e36}.get(case, 1.0)
    c *= scale
    if case == "mixed":
        c[rng.random(M) < 0.01] *= 1e8
    elif case == "sparse":
        c[rng.random(M) < 0.98] = 0
    c64 = c.astype(np.complex64)
    p = mn.Type1PlanND(tuple(x), (64, 64, 48), eps=1e-5)
    assert p.pts.kind == "zsweep" and p.w == 6
    g = torch.empty(p.n_up, dtype=torch.complex64, device="cuda")
    E.spread_zsweep(p.pts, p.beta, torch.from_numpy(c64).cuda(), g)
    assert bool(torch.isfinite(torch.view_as_real(g)).all())
    i1o, fro = oracle.setpts_t12(x, p.n_up, p.w)
    go = oracle.spread(i1o, fro, c64, p.n_up, p.w, p.beta)
    err = oracle.rel_l2(g.cpu().numpy().astype(np.complex128), go)
    print(f"  vs oracle: {err:.2e}")
    assert err < 1e-5


@pytest.mark.parametrize("B,presorted", [(1, False), (2, False), (3, True), (5, False)])
def test_zsweep_batch(B, presorted, oracle, mn, monkeypatch):
    """Batched z-sweep (vector pairs in 32-point batches, an odd last vector
    on its own) against the one-vector spread of every vector, whatever the
    vectors' magnitudes: the pair kernel sums the same products per
    accumulator in other K-steps, so the grids agree to fp32 rounding (rel
    l2 below 2e-7, each vector scaled on its own); with pairs switched off
    (MN_ZSWEEP_PAIRS=0) they are bit-identical. Every vector also against
    the oracle's fp64 spread."""
    from mlx_nufft_amd import _engine as E

    print(f"case zsweep batch B={B} presorted={presorted}", flush=True)
    rng = np.random.default_rng(40 + B)
    M, N = 30_000, (32, 40, 36)
    x = [rng.uniform(-np.pi, np.pi, M) for _ in range(3)]
    x[2][: M // 3] = rng.uniform(-0.2, 0.2, M // 3)   # a dense slab: full batches
    p = mn.Type1PlanND(tuple(x), N, eps=1e-5)
    assert p.pts.kind == "zsweep"
    scales = [1.0, 1e-30, 1e30, 3e-3, 7.0]
    cs = np.stack([(rng.standard_normal(M) + 1j * rng.standard_normal(M)) * scales[b]
                   for b in range(B)]).astype(np.complex64)
    cs[B - 1, ::7] = 0
    cd = torch.from_numpy(cs).cuda()
    if presorted:
        cd = cd[:, p.pts.perm.long()].contiguous()
    grids = torch.full((B, *p.n_up), float("nan"), dtype=torch.complex64, device="cuda")
    E.spread_zsweep_batch(p.pts, p.beta, cd, grids, presorted=presorted)
    monkeypatch.setenv("MN_ZSWEEP_PAIRS", "0")
    solo = torch.full((B, *p.n_up), float("nan"), dtype=torch.complex64, device="cuda")
    E.spread_zsweep_batch(p.pts, p.beta, cd, solo, presorted=presorted)
    monkeypatch.delenv("MN_ZSWEEP_PAIRS")
    one = torch.empty(p.n_up, dtype=torch.complex64, device="cuda")
    i1o, fro = oracle.setpts_t12(x, p.n_up, p.w)
    for b in range(B):
        one.fill_(float("nan"))
        E.spread_zsweep(p.pts, p.beta, cd[b].contiguous(), one, presorted=presorted)
        assert torch.equal(solo[b].view(torch.int64), one.view(torch.int64)), b
        assert bool(torch.isfinite(torch.view_as_real(grids[b])).all()), b
        g64, o64 = grids[b].to(torch.complex128), one.to(torch.complex128)  # 1e+-30 scales
        d = float((g64 - o64).abs().norm() / o64.abs().norm())
        assert d < 2e-7, (b, d)
        go = oracle.spread(i1o, fro, cs[b], p.n_up, p.w, p.beta)
        assert oracle.rel_l2(grids[b].cpu().numpy(), go) < 1e-5, b


def test_execute_batch_3d(oracle, mn):
    """Type-1 execute_batch in 3D against execute per vector and the direct
    sum (ref: nd.py:744-794)."""
    print("case execute_batch 3D", flush=True)
    rng = np.random.default_rng(47)
    M, N, B, eps = 8000, (16, 20, 12), 3, 1e-6
    x = [rng.uniform(-np.pi, np.pi, M) for _ in range(3)]
    cs = (rng.standard_normal((B, M)) + 1j * rng.standard_normal((B, M))).astype(np.complex64)
    p = mn.Type1PlanND(tuple(x), N, eps=eps)
    assert p.pts.kind == "zsweep"
    fb = p.execute_batch(cs)
    assert fb.shape == (B, *N)
    modes = [np.arange(-(n // 2), n - n // 2) for n in N]
    for b in range(B):
        assert oracle.rel_l2(fb[b], p.execute(cs[b])) < 1e-6
        assert oracle.rel_l2(fb[b], oracle.dft_t1(x, cs[b], modes, +1)) < 1e-5
