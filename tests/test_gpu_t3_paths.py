"""GPU checks of the type-3 execution paths and the kernels behind them.

* the fp64 zero-padding line FFT (mn_fft64_lines): one pass against numpy's
  FFT of the explicitly padded, deconvolved lines, for every radix (2, 3,
  4, 5, 8 and mixes), odd and even nin, nin = 1 and nin = n, contiguous
  (B = 1) and strided (B > 1) lines, partial last tiles, both signs and
  both output precisions; three passes (z, y, x) against numpy's ifftn /
  fftn of the padded grid; invalid lengths and shapes raise;
* type-3 through the line passes equals type-3 through pad + rocFFT, and
  matches the direct sum;
* the owner-computes fp64 spread equals the LDS-tile fp64 spread on awkward
  grids (partial and wrapping bins, w up to 16, clustered points), in
  isolation and through the type-3 plan, and the plan's spread selection;
* the direct gather equals the staged gather and the oracle's fp64 interp
  (footprints wrapping on every face), and the plan's gather selection;
* moving sources: set_sources within a planned source_extent (P changing,
  both backends, both spreads) equals a fresh plan, and sources past the
  extent's guard band raise.
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _padded(x, dec, n):
    """(A, nin, B) -> (A, n, B): element m times dec[m] at (m - nin//2) mod n."""
    A, nin, B = x.shape
    pos = (np.arange(nin) - nin // 2) % n
    out = np.zeros((A, n, B), np.complex128)
    out[:, pos, :] = x * (dec[None, :, None] if dec is not None else 1.0)
    return out


def _ref(x, dec, n, isign):
    p = _padded(x, dec, n)
    return np.fft.ifft(p, axis=1) * n if isign > 0 else np.fft.fft(p, axis=1)


CASES = [  # (A, nin, B, n)
    (7, 18, 1, 24), (3, 5, 7, 8), (1, 1, 33, 2), (2, 3, 5, 3), (4, 5, 3, 5),
    (5, 13, 1, 16), (3, 40, 9, 64), (2, 25, 6, 30), (1, 180, 17, 240), (9, 486, 1, 640),
    (1, 639, 8, 640), (3, 625, 2, 625), (2, 729, 3, 729), (1, 5760, 3, 7200),
    (2, 8192, 1, 8192), (1, 4001, 2, 4096), (300, 7, 1, 12), (1, 90, 1000, 120),
    # unpadded tiles of strided lines: 8 (n = 640, 512, 486), 16 (n = 320,
    # 256) and 32 (n = 160) lines
    (2, 486, 16, 640), (1, 400, 64, 512), (3, 480, 8, 486), (2, 300, 32, 320),
    (1, 200, 64, 256), (2, 150, 64, 160),
]


@pytest.mark.parametrize("A,nin,B,n", CASES)
@pytest.mark.parametrize("isign", [+1, -1])
def test_fft64_lines_vs_numpy(A, nin, B, n, isign, mn):
    from mlx_nufft_amd import _engine as E

    print(f"case fft64_lines A={A} nin={nin} B={B} n={n} isign={isign}", flush=True)
    rng = np.random.default_rng(n * 7 + nin)
    x = rng.standard_normal((A, nin, B)) + 1j * rng.standard_normal((A, nin, B))
    dec = rng.uniform(0.5, 2.0, nin)
    ref = _ref(x, dec, n, isign)
    xd = torch.from_numpy(x).cuda()
    dd = torch.from_numpy(dec).cuda()
    out = torch.full((A, n, B), complex(np.nan, np.nan), dtype=torch.complex128, device="cuda")
    E.fft64_lines(A, nin, B, n, isign, xd, dd, out)
    got = out.cpu().numpy()
    err = np.abs(got - ref).max() / np.abs(ref).max()
    assert err < 1e-13, err
    out32 = torch.empty((A, n, B), dtype=torch.complex64, device="cuda")
    E.fft64_lines(A, nin, B, n, isign, xd, None, out32)
    ref32 = _ref(x, None, n, isign)
    err32 = np.abs(out32.cpu().numpy() - ref32).max() / np.abs(ref32).max()
    assert err32 < 1e-6, err32


@pytest.mark.parametrize("nf,nu", [((18, 20, 10), (24, 30, 16)), ((45, 36, 18), (60, 48, 24)),
                                   ((7, 9, 11), (8, 10, 12))])
@pytest.mark.parametrize("isign", [+1, -1])
def test_fft64_lines_three_passes_vs_fftn(nf, nu, isign, mn):
    from mlx_nufft_amd import _engine as E

    print(f"case fft64_lines 3D nf={nf} nu={nu} isign={isign}", flush=True)
    rng = np.random.default_rng(sum(nf))
    bf = rng.standard_normal(nf) + 1j * rng.standard_normal(nf)
    decs = [rng.uniform(0.5, 2.0, k) for k in nf]
    pad = np.zeros(nu, np.complex128)
    idx = np.ix_(*[(np.arange(k) - k // 2) % n for k, n in zip(nf, nu)])
    pad[idx] = bf * decs[0][:, None, None] * decs[1][None, :, None] * decs[2][None, None, :]
    ref = np.fft.ifftn(pad) * np.prod(nu) if isign > 0 else np.fft.fftn(pad)
    bd = torch.from_numpy(bf).cuda()
    dd = [torch.from_numpy(d).cuda() for d in decs]
    T1 = torch.empty((nf[0], nf[1], nu[2]), dtype=torch.complex128, device="cuda")
    T2 = torch.empty((nf[0], nu[1], nu[2]), dtype=torch.complex128, device="cuda")
    H = torch.empty(nu, dtype=torch.complex128, device="cuda")
    E.fft64_lines(nf[0] * nf[1], nf[2], 1, nu[2], isign, bd, dd[2], T1)
    E.fft64_lines(nf[0], nf[1], nu[2], nu[1], isign, T1, dd[1], T2)
    E.fft64_lines(1, nf[0], nu[1] * nu[2], nu[0], isign, T2, dd[0], H)
    err = np.abs(H.cpu().numpy() - ref).max() / np.abs(ref).max()
    assert err < 1e-13, err
    # the type-3 plan's x pass: whole lines, the grid as (n1, n2, n0)
    Hl = torch.empty((nu[1], nu[2], nu[0]), dtype=torch.complex128, device="cuda")
    E.fft64_lines(1, nf[0], nu[1] * nu[2], nu[0], isign, T2, dd[0], Hl, layout="lines_first")
    errl = np.abs(Hl.cpu().numpy() - np.transpose(ref, (1, 2, 0))).max() / np.abs(ref).max()
    assert errl < 1e-13, errl


@pytest.mark.parametrize("A,nin,B,n", [(7, 18, 1, 24), (300, 18, 1, 24), (6, 5, 4, 8),
                                        (2, 486, 1, 640), (1, 30, 64, 40)])
def test_fft64_lines_lines_last(A, nin, B, n, mn):
    """lines_last: the same transform written as (n, A*B), line index fastest."""
    from mlx_nufft_amd import _engine as E

    print(f"case fft64_lines lines_last A={A} nin={nin} B={B} n={n}", flush=True)
    rng = np.random.default_rng(A + nin + B + n)
    x = rng.standard_normal((A, nin, B)) + 1j * rng.standard_normal((A, nin, B))
    dec = rng.uniform(0.5, 2.0, nin)
    ref = _ref(x, dec, n, +1)                                 # (A, n, B)
    ref_t = np.transpose(ref, (1, 0, 2)).reshape(n, A * B)   # (n, lines)
    out = torch.full((n, A * B), complex(np.nan, np.nan), dtype=torch.complex128, device="cuda")
    E.fft64_lines(A, nin, B, n, +1, torch.from_numpy(x).cuda(), torch.from_numpy(dec).cuda(),
                  out, layout="lines_last")
    err = np.abs(out.cpu().numpy() - ref_t).max() / np.abs(ref_t).max()
    assert err < 1e-13, err


@pytest.mark.parametrize("A,nin,B,n", [(7, 18, 1, 24), (1, 18, 300, 24), (6, 5, 4, 8),
                                        (1, 486, 16, 640), (3, 30, 64, 40), (1, 50, 6, 5400)])
def test_fft64_lines_lines_first(A, nin, B, n, mn):
    """lines_first: the same transform written as (A*B, n), each line's
    values contiguous (strided input lines included), complex128 and
    complex64."""
    from mlx_nufft_amd import _engine as E

    print(f"case fft64_lines lines_first A={A} nin={nin} B={B} n={n}", flush=True)
    rng = np.random.default_rng(A + nin + B + n + 1)
    x = rng.standard_normal((A, nin, B)) + 1j * rng.standard_normal((A, nin, B))
    dec = rng.uniform(0.5, 2.0, nin)
    ref = _ref(x, dec, n, -1)                                 # (A, n, B)
    ref_l = np.transpose(ref, (0, 2, 1)).reshape(A * B, n)    # (lines, n)
    xd, dd = torch.from_numpy(x).cuda(), torch.from_numpy(dec).cuda()
    out = torch.full((A * B, n), complex(np.nan, np.nan), dtype=torch.complex128, device="cuda")
    E.fft64_lines(A, nin, B, n, -1, xd, dd, out, layout="lines_first")
    err = np.abs(out.cpu().numpy() - ref_l).max() / np.abs(ref_l).max()
    assert err < 1e-13, err
    out32 = torch.full((A * B, n), complex(np.nan, np.nan), dtype=torch.complex64, device="cuda")
    E.fft64_lines(A, nin, B, n, -1, xd, dd, out32, layout="lines_first")
    err32 = np.abs(out32.cpu().numpy() - ref_l).max() / np.abs(ref_l).max()
    assert err32 < 1e-6, err32


@pytest.mark.parametrize("Bt,R,C", [(1, 1, 1), (3, 37, 70), (24, 64, 96), (2, 200, 33)])
def test_transpose_c128(Bt, R, C, mn):
    from mlx_nufft_amd import _engine as E

    print(f"case transpose Bt={Bt} R={R} C={C}", flush=True)
    rng = np.random.default_rng(R * C + Bt)
    a = rng.standard_normal((Bt, R, C)) + 1j * rng.standard_normal((Bt, R, C))
    out = torch.full((Bt, C, R), complex(np.nan, np.nan), dtype=torch.complex128, device="cuda")
    E.transpose_c128(Bt, R, C, torch.from_numpy(a).cuda(), out)
    assert np.array_equal(out.cpu().numpy(), np.transpose(a, (0, 2, 1)))


def test_fft64_lines_rejects_bad_shapes(mn):
    from mlx_nufft_amd import _engine as E
    from mlx_nufft_amd import _lib as L

    print("case fft64_lines errors", flush=True)
    for n, ok in [(7, False), (14, False), (8194, False), (10800, False), (8192, True),
                  (7200, True), (1, False), (2, True)]:
        assert E.fft64_lines_supported(n) == ok, n
    x = torch.zeros((2, 8, 1), dtype=torch.complex128, device="cuda")
    out = torch.zeros((2, 16, 1), dtype=torch.complex128, device="cuda")
    with pytest.raises(ValueError):
        E.fft64_lines(2, 8, 1, 14, +1, x, None, out)     # 14 = 2 * 7
    with pytest.raises(ValueError):
        L.check(L.lib().mn_fft64_lines(2, 17, 1, 16, 1, L.ptr(x), None, L.ptr(out), 0, 0,
                                       L.stream()), "nin > n")
    with pytest.raises(ValueError):
        L.check(L.lib().mn_fft64_lines(2, 8, 1, 16, 1, L.ptr(x), None, L.ptr(x), 0, 0,
                                       L.stream()), "aliasing")
    with pytest.raises(ValueError):
        L.check(L.lib().mn_transpose_c128(2, 4, 4, L.ptr(x), L.ptr(x), L.stream()), "aliasing")


def _gen_generic(P, M, X, S, seed):
    rng = np.random.default_rng(seed)
    x = tuple(rng.uniform(-X, X, P) for _ in range(3))
    s = tuple(rng.uniform(-S, S, M) for _ in range(3))
    c = rng.standard_normal(P) + 1j * rng.standard_normal(P)
    return x, c, s


@pytest.mark.parametrize("X,S", [(1.0, 200.0), (30.0, 20.0), (5.0, 9.0)])
@pytest.mark.parametrize("isign", [+1, -1])
def test_type3_lines_equals_rocfft_path(X, S, isign, oracle, mn, monkeypatch):
    print(f"case t3 lines vs rocfft X={X} S={S} isign={isign}", flush=True)
    x, c, s = _gen_generic(60_000, 40_000, X, S, seed=int(X * S))
    pl = mn.Type3Plan(x, s, eps=1e-5, isign=isign)
    assert pl.fft_lines
    fl = pl.execute(c.astype(np.complex64))
    monkeypatch.setenv("MN_T3_FFT", "rocfft")
    pr = mn.Type3Plan(x, s, eps=1e-5, isign=isign)
    assert not pr.fft_lines
    fr = pr.execute(c.astype(np.complex64))
    # the inner grids: the line passes store theirs as (n1, n2, n0), x
    # innermost; both are fp64 transforms rounded to complex64
    hl = np.transpose(pl._H.cpu().numpy(), (2, 0, 1))
    hr = pr._H.cpu().numpy()
    assert np.abs(hl - hr).max() <= 2.0 ** -22 * np.abs(hr).max()
    # the gathers sum the same taps in another axis order (x innermost on
    # the line-pass grid); cancellation at the band edges, which the post
    # factor scales up, makes that fp32 rounding visible at about 2.5e-6
    assert oracle.rel_l2(fl, fr) < 1e-5
    idx = np.random.default_rng(1).choice(s[0].size, 500, replace=False)
    fd = oracle.dft_t3(x, c, s, isign, idx=idx)
    err = oracle.rel_l2(fl[idx], fd)
    print(f"  n_up={pl.n_up} rel_l2={err:.3e}", flush=True)
    assert err < 1e-4


@pytest.mark.parametrize("n,w,clustered", [
    ((40, 36, 33), 9, False),   # partial last bins; 36: reaching bins wrap into one another
    ((50, 48, 20), 8, True),    # a 2-cell last bin; points packed at the periodic corner
    ((16, 18, 17), 16, False),  # w = 16, bins of 16 and one-cell last bins
    ((64, 64, 64), 2, False),
    ((12, 30, 96), 6, True),    # a dim narrower than a bin (one bin)
])
def test_spread_owner_equals_tiles(n, w, clustered, mn):
    """The owner-computes fp64 spread against the LDS-tile fp64 spread on the
    same sorted points (two independent accumulations of the same taps)."""
    from mlx_nufft_amd import _engine as E
    from mlx_nufft_amd import _lib as L

    print(f"case spread_owner n={n} w={w} clustered={clustered}", flush=True)
    rng = np.random.default_rng(sum(n) + w)
    P = 30_000
    beta = 2.3 * w
    if clustered:
        i1 = np.stack([(-w // 2 + rng.integers(-3, 4, P)) % k for k in n])
    else:
        i1 = np.stack([rng.integers(-w, k, P) for k in n])
    fr = rng.uniform(0, 1, (3, P)).astype(np.float32)
    c = torch.from_numpy((rng.standard_normal(P) + 1j * rng.standard_normal(P))
                         .astype(np.complex64)).cuda()
    pre = torch.from_numpy(np.exp(1j * rng.uniform(0, 6.3, P)).astype(np.complex64)).cuda()
    i1d = torch.from_numpy(i1.astype(np.int32)).cuda()
    frd = torch.from_numpy(fr).cuda()

    def keys(bins):
        hw = w // 2
        k = np.zeros(P, np.int64)
        for d in range(3):
            k = k * bins.nb[d] + ((i1[d] + hw) % n[d]) // bins.m[d]
        return torch.from_numpy(k.astype(np.int32)).cuda()

    bo = E.make_bins(3, w, n, m=[min(E.OWNER_M, k) for k in n])
    po = E.SortedPoints(bo, i1d, frd, keys(bo), stream=True)
    go = torch.full(n, complex(np.nan, np.nan), dtype=torch.complex128, device="cuda")
    # pre is in sorted order in both paths: gather it by each sort's perm
    E.spread_owner_c128(po, beta, c, go, pre=pre[po.perm.long()])
    bt = E.make_bins(3, w, n, cell_bytes=E.SPREAD_CELL_BYTES)
    pt = E.SortedPoints(bt, i1d, frd, keys(bt))
    gt = torch.empty(n, dtype=torch.complex128, device="cuda")
    E.spread_c128(pt, beta, c, gt, pre=pre[pt.perm.long()])
    a, b = go.cpu().numpy(), gt.cpu().numpy()
    assert np.isfinite(a).all()
    err = np.abs(a - b).max() / np.abs(b).max()
    assert err < 1e-12, err
    assert L.lib().mn_spread_owner_c128 is not None


@pytest.mark.parametrize("n,w,clustered,P,use_pre", [
    ((40, 36, 33), 9, False, 30_000, True),  # partial last bins (m = 8)
    ((50, 48, 20), 8, True, 30_000, True),   # points packed at the periodic corner
    ((16, 18, 17), 16, False, 5_000, True),  # w = 16: one-cell bins, tiles of 16
    ((64, 64, 64), 2, False, 50_000, True),  # bins of 15
    ((12, 30, 7), 6, True, 20_000, True),    # dims narrower than a bin (tiles under 16)
    ((24, 24, 24), 9, True, 3_000, True),    # clustered: subproblems split at 1024 points
    ((32, 40, 24), 7, False, 20_000, False),  # no prephase (a NULL pre pointer)
])
def test_spread_tile_mfma_equals_lds_tiles(n, w, clustered, P, use_pre, mn, monkeypatch):
    """The matrix-core fp64 tile spread against the LDS-atomic fp64 tile
    spread on the same sorted points and bins (type-3 tile bins: padded tiles
    of at most 16 cells), and against the owner-computes spread on its
    matrix-core and LDS-atomic kernels (owner bins of at most 16 cells):
    four independent fp64 accumulations of the same taps. The owner grids
    start as NaN, so a cell the owner kernel left unwritten fails."""
    from mlx_nufft_amd import _engine as E

    print(f"case spread tile mfma n={n} w={w} clustered={clustered} P={P} pre={use_pre}",
          flush=True)
    rng = np.random.default_rng(sum(n) * 7 + w)
    beta = 2.3 * w
    if clustered:
        i1 = np.stack([(-w // 2 + rng.integers(-2, 3, P)) % k for k in n])
    else:
        i1 = np.stack([rng.integers(-w, k, P) for k in n])
    fr = rng.uniform(0, 1, (3, P)).astype(np.float32)
    c = torch.from_numpy((rng.standard_normal(P) + 1j * rng.standard_normal(P))
                         .astype(np.complex64)).cuda()
    pre = torch.from_numpy(np.exp(1j * rng.uniform(0, 6.3, P)).astype(np.complex64)).cuda()
    i1d = torch.from_numpy(i1.astype(np.int32)).cuda()
    frd = torch.from_numpy(fr).cuda()
    bt = E.t3_tile_bins(w, n)
    assert all(bt.m[d] + w - 1 <= 16 for d in range(3))
    hw = w // 2
    k = np.zeros(P, np.int64)
    for d in range(3):
        k = k * bt.nb[d] + ((i1[d] + hw) % n[d]) // bt.m[d]
    pt = E.SortedPoints(bt, i1d, frd, torch.from_numpy(k.astype(np.int32)).cuda())
    pre_s = pre[pt.perm.long()] if use_pre else None
    g_mfma = torch.full(n, complex(np.nan, np.nan), dtype=torch.complex128, device="cuda")
    E.spread_c128(pt, beta, c, g_mfma, pre=pre_s)
    monkeypatch.setenv("MN_T3_TILE_MFMA", "0")
    g_lds = torch.full(n, complex(np.nan, np.nan), dtype=torch.complex128, device="cuda")
    E.spread_c128(pt, beta, c, g_lds, pre=pre_s)
    monkeypatch.delenv("MN_T3_TILE_MFMA")
    bo = E.make_bins(3, w, n, m=[min(E.OWNER_M, kk) for kk in n])
    kk = np.zeros(P, np.int64)
    for d in range(3):
        kk = kk * bo.nb[d] + ((i1[d] + hw) % n[d]) // bo.m[d]
    po = E.SortedPoints(bo, i1d, frd, torch.from_numpy(kk.astype(np.int32)).cuda(), stream=True)
    g_own = torch.full(n, complex(np.nan, np.nan), dtype=torch.complex128, device="cuda")
    pre_o = pre[po.perm.long()] if use_pre else None
    E.spread_owner_c128(po, beta, c, g_own, pre=pre_o)
    monkeypatch.setenv("MN_T3_OWNER_MFMA", "0")
    g_own_lds = torch.full(n, complex(np.nan, np.nan), dtype=torch.complex128, device="cuda")
    E.spread_owner_c128(po, beta, c, g_own_lds, pre=pre_o)
    monkeypatch.delenv("MN_T3_OWNER_MFMA")
    a, b = g_mfma.cpu().numpy(), g_lds.cpu().numpy()
    o, ol = g_own.cpu().numpy(), g_own_lds.cpu().numpy()
    assert np.isfinite(a).all() and np.isfinite(b).all()
    assert np.isfinite(o).all() and np.isfinite(ol).all()
    scale = np.abs(b).max()
    assert np.abs(a - b).max() / scale < 1e-13
    assert np.abs(a - o).max() / scale < 1e-13
    assert np.abs(o - ol).max() / scale < 1e-13


def test_type3_owner_equals_tiles_spread(oracle, mn, monkeypatch):
    """Type-3 through each spread (forced), equal to within the c64 rounding."""
    print("case t3 owner vs tiles spread", flush=True)
    x, c, s = _gen_generic(80_000, 30_000, 8.0, 12.0, seed=3)
    monkeypatch.setenv("MN_T3_SPREAD", "owner")
    po = mn.Type3Plan(x, s, eps=1e-6, isign=-1)
    assert po.spread_owner
    fo = po.execute(c.astype(np.complex64))
    monkeypatch.setenv("MN_T3_SPREAD", "tiles")
    pt = mn.Type3Plan(x, s, eps=1e-6, isign=-1)
    assert not pt.spread_owner
    ft = pt.execute(c.astype(np.complex64))
    assert oracle.rel_l2(fo, ft) < 1e-6


def test_type3_spread_selection(mn, monkeypatch):
    """The automatic choice: owner spread for mid-density isotropic grids,
    tiles for dense grids and thin slabs; MN_T3_SPREAD overrides."""
    print("case t3 spread selection", flush=True)
    x, c, s = _gen_generic(100_000, 2_000, 30.0, 20.0, seed=4)   # 486^3-class grid, 0.4 taps/cell
    assert mn.Type3Plan(x, s, eps=3e-5).spread_owner
    x, c, s = _gen_generic(200_000, 2_000, 1.0, 60.0, seed=5)    # dense: ~60^3 grid
    assert not mn.Type3Plan(x, s, eps=1e-5).spread_owner
    monkeypatch.setenv("MN_T3_SPREAD", "owner")
    assert mn.Type3Plan(x, s, eps=1e-5).spread_owner
    monkeypatch.setenv("MN_T3_SPREAD", "bogus")
    with pytest.raises(ValueError):
        mn.Type3Plan(x, s, eps=1e-5)


@pytest.mark.parametrize("n,w", [((40, 36, 24), 9), ((16, 16, 16), 16), ((64, 48, 33), 6),
                                 ((9, 12, 10), 9)])
def test_interp_direct_equals_tiles(n, w, oracle, mn):
    """Direct gather against the staged-tile gather and the oracle's fp64
    interp on the same points, footprints wrapping on every face."""
    from mlx_nufft_amd import _engine as E

    print(f"case interp_direct n={n} w={w}", flush=True)
    rng = np.random.default_rng(sum(n) * w)
    P, beta = 20_000, 2.3 * w
    i1 = np.stack([rng.integers(-(w // 2), k, P) for k in n]).astype(np.int32)
    fr = rng.uniform(0, 1, (3, P)).astype(np.float32)
    grid = (rng.standard_normal(n) + 1j * rng.standard_normal(n)).astype(np.complex64)
    post = np.exp(1j * rng.uniform(0, 6.3, P)).astype(np.complex64)
    hw = w // 2
    bins = E.make_bins(3, w, n, cell_bytes=E.INTERP_CELL_BYTES)
    k = np.zeros(P, np.int64)
    for d in range(3):
        k = k * bins.nb[d] + ((i1[d] + hw) % n[d]) // bins.m[d]
    pts = E.SortedPoints(bins, torch.from_numpy(i1).cuda(), torch.from_numpy(fr).cuda(),
                         torch.from_numpy(k.astype(np.int32)).cuda())
    gd = torch.from_numpy(grid).cuda()
    ps = torch.from_numpy(post).cuda()[pts.perm.long()]
    od = torch.full((P,), complex(np.nan, np.nan), dtype=torch.complex64, device="cuda")
    ot = torch.empty(P, dtype=torch.complex64, device="cuda")
    E.interp_direct(pts, beta, gd, od, post=ps)
    E.interp(pts, beta, gd, ot, post=ps)
    a, b = od.cpu().numpy(), ot.cpu().numpy()
    assert np.isfinite(a).all()
    assert oracle.rel_l2(a, b) < 1e-6
    ref = oracle.interp(i1, fr, grid, w, beta) * post
    # fp32 weights and sums over w^3 taps against the fp64 oracle (1.5e-6 at w = 16)
    assert oracle.rel_l2(a, ref) < 4e-6


def test_type3_direct_gather_selection(oracle, mn, monkeypatch):
    """Sparse targets on a large grid take the direct gather, dense ones the
    staged gather; forced staged and direct agree."""
    print("case t3 gather selection", flush=True)
    x, c, s = _gen_generic(50_000, 20_000, 30.0, 20.0, seed=6)
    pa = mn.Type3Plan(x, s, eps=1e-5)
    assert pa.gather_direct
    fa = pa.execute(c.astype(np.complex64))
    monkeypatch.setenv("MN_T3_GATHER", "staged")
    pb = mn.Type3Plan(x, s, eps=1e-5)
    assert not pb.gather_direct
    fb = pb.execute(c.astype(np.complex64))
    # two fp32 gathers in different summation orders, then the target
    # deconvolution 1/phihat(theta) (~1e2 at the band edges): ~3e-6 apart
    assert oracle.rel_l2(fa, fb) < 1e-5
    idx = np.random.default_rng(2).choice(s[0].size, 400, replace=False)
    assert oracle.rel_l2(fa[idx], oracle.dft_t3(x, c, s, +1, idx=idx)) < 1e-4
    monkeypatch.delenv("MN_T3_GATHER")
    x, c, s = _gen_generic(2_000, 400_000, 1.0, 25.0, seed=7)    # 400k targets on ~30^3
    assert not mn.Type3Plan(x, s, eps=1e-5).gather_direct


def test_type3_reversed_axis_pipeline(oracle, mn, monkeypatch):
    """Grids with a long x or y axis take the reversed-axis line pipeline
    (z-pass written axis-outermost, contiguous y-pass, transpose, contiguous
    x-pass, targets gathered with their axes reversed); it equals the pad +
    rocFFT path and matches the direct sum."""
    import sys
    import pathlib
    sys.path.insert(0, str(pathlib.Path(__file__).parent))
    from test_gpu_t3_large import gen_anisotropic

    print("case t3 reversed-axis pipeline", flush=True)
    x, c, s = gen_anisotropic(64, 5_000, 0.5)
    for isign in (+1, -1):
        monkeypatch.delenv("MN_T3_FFT", raising=False)
        pl = mn.Type3Plan(x, s, eps=1e-5, isign=isign)
        assert pl.fft_lines and pl.fft_rev and max(pl.n_up[:2]) > 1365, pl.n_up
        fl = pl.execute(c.astype(np.complex64))
        monkeypatch.setenv("MN_T3_FFT", "rocfft")
        pr = mn.Type3Plan(x, s, eps=1e-5, isign=isign)
        assert not pr.fft_lines
        fr = pr.execute(c.astype(np.complex64))
        assert oracle.rel_l2(fl, fr) < 1e-5
        idx = np.random.default_rng(3).choice(s[0].size, 500, replace=False)
        err = oracle.rel_l2(fl[idx], oracle.dft_t3(x, c, s, isign, idx=idx))
        print(f"  isign={isign} n_up={pl.n_up} rel_l2={err:.3e}", flush=True)
        assert err < 1e-4


@pytest.mark.parametrize("spread", ["owner", "tiles"])
def test_type3_set_sources(spread, oracle, mn, monkeypatch):
    """Moving sources (ref: gpu_t3.py:444-506): a plan sized with
    source_extent takes new frames (P may change) and equals a fresh plan of
    the same extent; sources past the extent plus the guard band raise."""
    print(f"case t3 set_sources spread={spread}", flush=True)
    monkeypatch.setenv("MN_T3_SPREAD", spread)
    rng = np.random.default_rng(11)
    ext = [(-2.2, 2.2)] * 3
    s = tuple(rng.uniform(-15.0, 15.0, 20_000) for _ in range(3))
    x1 = tuple(rng.uniform(-2.0, 2.0, 30_000) for _ in range(3))
    p = mn.Type3Plan(x1, s, eps=1e-6, isign=-1, source_extent=ext)
    assert p.spread_owner == (spread == "owner")
    for P, backend in [(30_000, "host"), (45_000, "gpu"), (12_345, "host")]:
        x2 = tuple(rng.uniform(-2.2, 2.2, P) for _ in range(3))
        c2 = (rng.standard_normal(P) + 1j * rng.standard_normal(P)).astype(np.complex64)
        p.set_sources(x2, backend=backend)
        assert p.P == P
        f = p.execute(c2)
        fresh = mn.Type3Plan(x2, s, eps=1e-6, isign=-1, source_extent=ext).execute(c2)
        assert oracle.rel_l2(f, fresh) < 1e-6
        idx = np.random.default_rng(P).choice(s[0].size, 300, replace=False)
        err = oracle.rel_l2(f[idx], oracle.dft_t3(x2, c2, s, -1, idx=idx))
        print(f"  P={P} backend={backend} rel_l2={err:.3e}", flush=True)
        assert err < 1e-4
    far = tuple(v.copy() for v in x1)
    far[1][7] = 3.5  # past 2.2 + guard
    with pytest.raises(ValueError):
        p.set_sources(far)
    with pytest.raises(ValueError):
        p.set_sources(x1, backend="cuda")


@pytest.mark.parametrize("prec", ["crit64", "coords64", "phases64", "fp32"])
def test_type3_setup_bit_exact(prec, oracle, mn):
    """Type-3 point setup against the oracle's restatement of the
    reference's host path (ref: gpu_t3.py:326-377, 474-488), in every
    precision mode: the plan's sizing scalars equal the oracle's exactly;
    the unsorted source and target cells and fractions that
    mn_t3_setpts_src / mn_t3_setpts_trg write are bit-identical, and the
    bin keys equal the key definition; pre and post agree to complex64
    rounding (their sincos and quadrature sums are fp64 in a different
    order). The sets hold exact ties (a source at the centre C gives
    xi - w/2 an integer; a target at D gives lam - w/2 an integer) and the
    sources that fix the extent."""
    import ctypes

    from mlx_nufft_amd import _lib as L
    from mlx_nufft_amd.sizing import quadrature

    rng = np.random.default_rng(44)
    P, M = 20000, 12000
    x = [1.5 * d + rng.uniform(-1, 1, P) for d in range(3)]
    s = [30.0 * (d - 1) + rng.uniform(-80, 80, M) for d in range(3)]
    for d in range(3):
        lo, hi = x[d][16:].min(), x[d][16:].max()
        x[d][:4] = [lo, hi, 0.5 * (lo + hi), 0.5 * (lo + hi)]   # extent edges and centre
        x[d][4:16] = lo + (hi - lo) * np.arange(1, 13) / 13.0
        slo, shi = s[d][4:].min(), s[d][4:].max()
        s[d][:4] = [slo, shi, 0.5 * (slo + shi), 0.5 * (slo + shi)]
    for isign, eps in ((+1, 1e-5), (-1, 3e-5)):   # w = 9 and w = 8
        print(f"case t3 setup prec={prec} isign={isign} eps={eps}", flush=True)
        st = oracle.t3_setup(x, s, eps, isign, 1.25, prec)
        plan = mn.Type3Plan(x, s, eps=eps, isign=isign, prec=prec)
        assert plan.nf == st["nf"] and plan.n_up == st["n_up"]
        assert plan.C == st["C"] and plan.D == st["D"] and plan.gam == st["gam"]
        assert not plan.fft_rev
        dev = torch.device("cuda")
        x64 = [torch.from_numpy(v).to(dev) for v in x]
        s64 = [torch.from_numpy(v).to(dev) for v in s]

        i1 = torch.empty((3, P), dtype=torch.int32, device=dev)
        fr = torch.empty((3, P), dtype=torch.float32, device=dev)
        key = torch.empty(P, dtype=torch.int32, device=dev)
        pre = torch.empty(P, dtype=torch.complex64, device=dev)
        hd = [2.0 * np.pi / n for n in st["nf"]]
        L.check(L.lib().mn_t3_setpts_src(
            ctypes.byref(plan.bins_src), P, L.ptr3(x64), L.d3(st["C"]), L.d3(st["gam"]),
            L.d3(hd), L.d3(st["D"]), isign, plan._flags, L.ptr3([i1[d] for d in range(3)]),
            L.ptr3([fr[d] for d in range(3)]), L.ptr(key), L.ptr(pre), L.stream()), "src")
        i1h, frh = i1.cpu().numpy(), fr.cpu().numpy()
        assert np.array_equal(i1h, st["i1"])
        assert np.array_equal(frh.view(np.int32), st["fr"].view(np.int32))
        g = plan.bins_src
        want_key, _ = oracle.bin_keys(st["i1"], st["nf"], [g.m[d] for d in range(3)], st["w"])
        assert np.array_equal(key.cpu().numpy().astype(np.int64), want_key.astype(np.int64))
        assert np.abs(pre.cpu().numpy() - st["pre"]).max() <= 1.2e-7
        # the plan's sorted state is a permutation of the same values
        perm = plan.src.perm.cpu().numpy().astype(np.int64)
        assert np.array_equal(plan.src.i1s.cpu().numpy(), st["i1"][:, perm])
        assert np.array_equal(plan.src.frs.cpu().numpy().view(np.int32),
                              st["fr"][:, perm].view(np.int32))

        ti1 = torch.empty((3, M), dtype=torch.int32, device=dev)
        tfr = torch.empty((3, M), dtype=torch.float32, device=dev)
        tkey = torch.empty(M, dtype=torch.int32, device=dev)
        post = torch.empty(M, dtype=torch.complex64, device=dev)
        dq, fq = quadrature(st["beta"], st["w"])
        quad = torch.from_numpy(np.concatenate([dq, fq])).to(dev)
        hg = [hd[d] * st["gam"][d] for d in range(3)]
        h2 = [2.0 * np.pi / n for n in st["n_up"]]
        L.check(L.lib().mn_t3_setpts_trg(
            ctypes.byref(plan.bins_trg), M, L.ptr3(s64), L.d3(st["D"]), L.d3(hg), L.d3(h2),
            L.d3(st["C"]), isign, plan._flags, L.ptr(quad), len(dq),
            L.ptr3([ti1[d] for d in range(3)]), L.ptr3([tfr[d] for d in range(3)]), L.ptr(tkey),
            L.ptr(post), L.stream()), "trg")
        assert np.array_equal(ti1.cpu().numpy(), st["t_i1"])
        assert np.array_equal(tfr.cpu().numpy().view(np.int32), st["t_fr"].view(np.int32))
        gt = plan.bins_trg
        want_tkey, _ = oracle.bin_keys(st["t_i1"], st["n_up"], [gt.m[d] for d in range(3)],
                                       st["w"])
        assert np.array_equal(tkey.cpu().numpy().astype(np.int64), want_tkey.astype(np.int64))
        ph = post.cpu().numpy()
        assert np.all(np.abs(ph - st["post"]) <= 2.5e-7 * np.abs(st["post"]))
        # the centre source: xi = nf/2 exactly, so i1 = ceil(nf/2 - w/2) and
        # fr = nf/2 - i1 (an exact tie, fr = w/2, when w is even); likewise
        # the target at D with lam = n_up/2
        for d in range(3):
            ci = int(np.ceil(st["nf"][d] / 2 - st["w"] / 2))
            assert i1h[d][2] == ci and frh[d][2] == st["nf"][d] / 2 - ci
            ti = int(np.ceil(st["n_up"][d] / 2 - st["w"] / 2))
            assert ti1.cpu().numpy()[d][2] == ti
        if st["w"] % 2 == 0:
            assert frh[0][2] == st["w"] / 2
