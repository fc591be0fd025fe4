"""Host-side checks that need no GPU.

* the C-ABI library loads and exports every function include/*.h declares,
  and the ctypes signature table covers exactly that set;
* the library's pure size queries (no device call);
* the product's sizing equals the oracle's (which tests/test_oracle.py pins);
* the engine's bin geometry and key widths;
* argument validation of the finufft-style surface, which raises before any
  device work, and the loud failure when no GPU is present (no CPU path).
"""

import ctypes
import pathlib
import re

import numpy as np
import pytest
import torch

ROOT = pathlib.Path(__file__).resolve().parents[1]


def _header_functions():
    names = []
    for h in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        names += re.findall(r"\b(mn_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


@pytest.fixture(scope="module")
def clib():
    from mlx_nufft_amd import _lib

    return _lib.load_library()


def test_header_symbols_exported(clib):
    from mlx_nufft_amd import _lib

    names = _header_functions()
    assert len(names) >= 25
    for n in names:
        assert hasattr(clib, n), f"{n} declared in include/ but not exported"
    assert sorted(_lib.EXPORTED) == names


def test_pure_queries(clib):
    from mlx_nufft_amd import _lib

    assert clib.mn_version() == 100
    ws = [clib.mn_sort_workspace_bytes(P) for P in (1, 1000, 1 << 20, 20_000_000)]
    assert all(b > 0 for b in ws) and ws == sorted(ws)
    # workspace holds at least the ping-pong key + perm buffers of P entries
    assert ws[-1] >= 2 * 4 * 20_000_000

    g = _lib.Bins.make(3, 6, [512, 512, 512], [8, 8, 1])
    assert clib.mn_zsweep_nkeys(ctypes.byref(g)) == 64 * 64 * 64 * 16
    # n2 not a multiple of 8: the last z-chunk is partial
    g = _lib.Bins.make(3, 6, [64, 64, 300], [8, 8, 1])
    assert clib.mn_zsweep_nkeys(ctypes.byref(g)) == 8 * 8 * 38 * 16
    # payload columns add one P-length alternate buffer each
    assert (clib.mn_sort_pairs_workspace_bytes(1 << 20, 3)
            >= clib.mn_sort_pairs_workspace_bytes(1 << 20, 0) + 3 * 4 * (1 << 20))
    assert clib.mn_sort_pairs_workspace_bytes(1000, 9) == -1
    # the z-sweep key space is capped at 2^23 keys
    assert clib.mn_zsweep_nkeys(ctypes.byref(_lib.Bins.make(3, 6, [1024, 1024, 256],
                                                            [8, 8, 1]))) == 1 << 23
    assert clib.mn_zsweep_nkeys(ctypes.byref(_lib.Bins.make(3, 6, [1024, 1024, 264],
                                                            [8, 8, 1]))) == -1
    assert clib.mn_subproblem_workspace_bytes(ctypes.byref(_lib.Bins.make(3, 6, [64] * 3,
                                                                          [11] * 3))) > 0
    # z-sweep geometry limits: w <= 8, n0 and n1 multiples of 8
    for bad in (_lib.Bins.make(3, 9, [512] * 3, [8, 8, 1]),
                _lib.Bins.make(3, 6, [500, 512, 512], [8, 8, 1]),
                _lib.Bins.make(2, 6, [512, 512], [8, 8])):
        assert clib.mn_zsweep_nkeys(ctypes.byref(bad)) == -1
        assert clib.mn_last_error().decode()
    # a grid smaller than the kernel width is rejected
    assert clib.mn_subproblem_workspace_bytes(ctypes.byref(_lib.Bins.make(1, 8, [6], [6]))) == -1


def test_bins_struct_layout():
    from mlx_nufft_amd import _lib

    # struct { int32 dim, w; int64 n[3]; int32 m[3], nb[3]; }
    assert ctypes.sizeof(_lib.Bins) == 8 + 24 + 12 + 12
    g = _lib.Bins.make(3, 6, [512, 480, 90], [11, 11, 11])
    assert list(g.nb) == [47, 44, 9] and g.nbins == 47 * 44 * 9


# ---------------------------------------------------------------- sizing --

def test_product_sizing_equals_oracle(oracle):
    from mlx_nufft_amd import sizing as S

    for n in list(range(0, 2000)) + [65537, 99991, 123457]:
        assert S.next235even(n) == oracle.next235even(n)
    for eps in (1e-1, 3e-2, 1e-3, 1e-4, 1e-5, 1e-6, 1e-7, 1e-9, 1e-12, 1e-15):
        for sig in (2.0, 1.25, 1.5):
            assert S.kernel_params(eps, sig) == oracle.kernel_params(eps, sig)
    xi = np.linspace(0, np.pi, 33)
    for w, beta in ((6, 13.8), (9, 16.45566231965758), (2, 4.4)):
        assert np.allclose(S.kernel_ft(xi, beta, w), oracle.kernel_ft(xi, beta, w),
                           rtol=1e-13, atol=0)
    for S_, X_ in ((200.0, 1.0), (0.0, 0.0), (30.0, 0.0), (0.0, 3.0), (1e4, 2.5)):
        assert S.set_nhg_type3(S_, X_, 1.25, 9) == pytest.approx(
            oracle.set_nhg_type3(S_, X_, 1.25, 9), rel=1e-15)


def test_engine_bin_geometry(monkeypatch):
    from mlx_nufft_amd import _engine as E

    monkeypatch.setattr(E, "_budget", 80 * 1024)
    monkeypatch.delenv("MN_BIN_M", raising=False)
    for w in range(2, 17):
        m = E.bin_sizes(3, w, [512] * 3)
        assert E.SPREAD_CELL_BYTES * np.prod([v + w - 1 for v in m]) <= 80 * 1024
        assert min(m) >= 1
    assert E.bin_sizes(1, 6, [8192]) == [1024]
    assert E.bin_sizes(2, 6, [20, 2048]) == [20, 32]
    assert E.zsweep_eligible(3, 6, [512, 512, 512])
    assert not E.zsweep_eligible(3, 9, [512, 512, 512])
    assert not E.zsweep_eligible(3, 6, [514, 512, 512])
    assert not E.zsweep_eligible(2, 6, [512, 512])
    assert E.zsweep_eligible(3, 6, [1024, 1024, 256])
    assert not E.zsweep_eligible(3, 6, [1024, 1024, 264])
    g = E.make_bins(3, 6, [512] * 3, m=(8, 8, 1))
    assert E.key_bits(g) == (64 * 64 * 512 - 1).bit_length()


def test_zsweep_class_ranks():
    """The z-sweep key's class ranking: for every width, the classes a
    neighbour's points must carry to reach a block (along x: cx > 0, along
    y: cy > 0, both for the -xy neighbour) are exactly the key-rank ranges
    the sweep reads, [3, 15), [0, 12) and [3, 12); a reach code is nonzero
    exactly when the footprint crosses into the next block."""
    from zsweep_words import rank, reach

    cx, cy = np.meshgrid(np.arange(4), np.arange(4), indexing="ij")
    r = rank(cx, cy)
    assert sorted(r.ravel()) == list(range(16))
    assert set(r[cx > 0]) == set(range(3, 15))
    assert set(r[cy > 0]) == set(range(0, 12))
    assert set(r[(cx > 0) & (cy > 0)]) == set(range(3, 12))
    for w in range(2, 9):
        o = np.arange(8)
        assert np.array_equal(reach(o, w) > 0, (o + w - 1) >= 8)
        # code 1 covers the lower half of the own block, 3 the upper half
        # of the next one
        assert np.array_equal(reach(o, w) == 1, ((o + w - 1) >= 8) & (o <= 3))
        assert np.array_equal(reach(o, w) == 3, (o + w - 1 >= 12) & (o > 3))


def test_checks_survive_python_O(tmp_path):
    """The size and option checks in front of raw device pointers (engine
    wrappers) and the type-3 plan options raise under python -O, which
    strips assert statements."""
    import subprocess
    import sys

    script = tmp_path / "checks.py"
    script.write_text(
        "import sys, torch\n"
        f"sys.path.insert(0, {str(ROOT)!r})\n"
        "from mlx_nufft_amd import _engine as E, t3\n"
        "def raises(fn, exc=ValueError):\n"
        "    try:\n"
        "        fn()\n"
        "    except exc:\n"
        "        return\n"
        "    raise SystemExit('no ' + exc.__name__ + ' from ' + repr(fn))\n"
        "c128 = torch.zeros(4, dtype=torch.complex128)\n"
        "raises(lambda: E.transpose_c128(2, 3, 4, c128, c128))\n"
        "raises(lambda: E.transpose_c128(1, 2, 2, c128, c128.to(torch.complex64)))\n"
        "raises(lambda: E.fft64_lines(2, 3, 4, 8, 1, c128, None, c128))\n"
        "class Pts:\n"
        "    P = 5\n"
        "cs = torch.zeros(2, 5, dtype=torch.complex64)\n"
        "g = torch.zeros(3, 4, 4, 4, dtype=torch.complex64)\n"
        "raises(lambda: E.spread_zsweep_batch(Pts(), 1.0, cs, g))\n"
        "x = [torch.zeros(3, dtype=torch.float64)] * 3\n"
        "raises(lambda: t3.GpuT3Plan(x, x, prec='fp16'))\n"
        "raises(lambda: t3.GpuT3Plan(x, x, fft_backend='cufft'))\n"
        "raises(lambda: t3.GpuT3Plan(x, x, prec='fp16'), AssertionError)\n"
        "print('ok')\n")
    out = subprocess.run([sys.executable, "-O", str(script)], capture_output=True, text=True,
                         timeout=300)
    assert out.returncode == 0 and out.stdout.strip().endswith("ok"), out.stdout + out.stderr


# ------------------------------------------------------------ validation --

def test_api_validation_errors(mn):
    x = np.zeros(10)
    with pytest.raises(NotImplementedError):
        mn.nufft1d1(x, x.astype(complex), 8, modeord=1)
    with pytest.raises(ValueError):
        mn.Plan(4, (8, 8))
    with pytest.raises(ValueError):
        mn.Plan(1, (8, 8), dtype="float64")
    with pytest.raises(ValueError):
        mn.Plan(1, (8, 8, 8, 8))
    with pytest.raises(ValueError):
        mn.Type1PlanND((x, x), (8, 8), prec="fp16")
    with pytest.raises(ValueError):
        mn.Type1PlanND((x, x), (8, 8, 8))
    with pytest.raises(ValueError):
        mn.Type1PlanND((x, x), (8, 0))
    with pytest.raises(ValueError):
        mn.Type1PlanND((x, x), (8, 8), upsampfac=5.0)
    with pytest.raises(ValueError):
        mn.Type1PlanND((x, x, x, x), 8)
    with pytest.raises(ValueError):
        mn.expi([np.zeros(3)] * 9)
    with pytest.raises(ValueError):
        mn.expi([np.zeros(3), np.zeros(4)])
    with pytest.raises(RuntimeError):
        mn.Type3Plan((x, x, x), (x, x, x), fft_backend="vkfft")
    assert mn.vkfft_available() is False
    p = mn.Plan(1, (8, 8))
    with pytest.raises(RuntimeError):
        p.execute(np.zeros(10, complex))


def test_spread_method_and_legacy_validation(mn):
    """Option checks that raise before any device work (ref: nd.py:281-305,
    397-404, 869-874; types12.py:36-37, 159-186)."""
    import inspect

    from mlx_nufft_amd.nd import PlanArgumentError, od_applicable

    x = np.zeros(10)
    for cls in (mn.Type1PlanND, mn.Type2PlanND):
        # an unknown method: a ValueError that is also the reference's
        # AssertionError
        for exc in (ValueError, AssertionError):
            with pytest.raises(exc):
                cls((x, x), (8, 8), spread_method="atomic")
        # a forced "od" outside the reference's output-driven rule
        with pytest.raises(ValueError, match="od"):
            cls((x, x), (64, 64), spread_method="od")            # P < 20000
        big = np.zeros(30000)
        with pytest.raises(ValueError, match="od"):
            cls((big, big), (64, 64), eps=1e-9, spread_method="od")   # w = 10 > 8
        with pytest.raises(ValueError, match="od"):
            cls((big,) * 3, (4, 4, 4), eps=1e-5, spread_method="od")   # grid 12^3 < tile 15^3
    # the rule itself, against the reference's tile sizes
    assert od_applicable(3, 6, [512] * 3, 20000)
    assert not od_applicable(3, 6, [512] * 3, 19999)
    assert not od_applicable(3, 9, [512] * 3, 10 ** 6)
    assert not od_applicable(3, 6, [14, 512, 512], 10 ** 6)
    assert od_applicable(3, 6, [15, 512, 512], 10 ** 6)
    assert od_applicable(2, 7, [48, 48], 10 ** 6) and not od_applicable(2, 7, [47, 48], 10 ** 6)
    assert od_applicable(1, 8, [2056], 10 ** 6) and not od_applicable(1, 8, [2055], 10 ** 6)

    # legacy plans: 3D, even mode sizes, and the reference's defaults
    for cls in (mn.Type1Plan, mn.Type2Plan):
        for bad in ((8, 8, 7), (8, 8), 9):
            with pytest.raises(PlanArgumentError):
                cls((x, x, x), bad)
        with pytest.raises(AssertionError):
            cls((x, x), (8, 8, 8))
        with pytest.raises(ValueError):
            cls((x, x, x), (8, 8, 8), prec="fp16")
    d1 = inspect.signature(mn.Type1Plan).parameters
    d2 = inspect.signature(mn.Type2Plan).parameters
    assert (d1["eps"].default, d1["isign"].default, d1["upsampfac"].default,
            d1["sort_points"].default) == (1e-5, 1, 1.25, True)
    assert (d2["eps"].default, d2["isign"].default, d2["upsampfac"].default,
            d2["sort_points"].default) == (1e-5, 1, 1.25, False)


def test_api_signatures(mn):
    """The finufft-style functions keep the reference's parameter names and
    defaults (ref: api.py:167-251, 258-260)."""
    import inspect

    want = {
        "nufft1d1": "x c n_modes out eps isign kwargs", "nufft2d1": "x y c n_modes out eps isign kwargs",
        "nufft3d1": "x y z c n_modes out eps isign kwargs", "nufft1d2": "x f out eps isign kwargs",
        "nufft2d2": "x y f out eps isign kwargs", "nufft3d2": "x y z f out eps isign kwargs",
        "nufft1d3": "x c s out eps isign kwargs", "nufft2d3": "x y c s t out eps isign kwargs",
        "nufft3d3": "x y z c s t u out eps isign kwargs",
    }
    for name, params in want.items():
        sig = inspect.signature(getattr(mn, name)).parameters
        assert " ".join(sig) == params, name
        assert sig["eps"].default == 1e-6 and sig["out"].default is None
        assert sig["isign"].default == (-1 if name[-1] == "2" else 1)
    ps = inspect.signature(mn.Plan).parameters
    assert (ps["n_trans"].default, ps["eps"].default, ps["isign"].default,
            ps["dtype"].default) == (1, 1e-6, None, "complex128")
    with pytest.warns(UserWarning, match="eps"):
        p = mn.Plan(1, (8, 8), eps=1e-9)
    assert p.eps == 1e-6 and p.isign == 1 and mn.Plan(2, 8).isign == -1
    with pytest.warns(UserWarning, match="unrecognised"):
        mn.Plan(1, (8, 8), bogus_option=3)
    mn.Plan(1, (8, 8), nthreads=4, spread_sort=2)   # finufft CPU options: silent


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU failure")
def test_no_gpu_fails_loudly(mn):
    """Without a ROCm device every compute entry raises; nothing falls back
    to a CPU implementation."""
    rng = np.random.default_rng(0)
    x = [rng.uniform(-np.pi, np.pi, 100) for _ in range(3)]
    c = np.ones(100, complex)
    for call in (lambda: mn.nufft3d1(*x, c, (8, 8, 8)),
                 lambda: mn.nufft2d2(x[0], x[1], np.ones((8, 8), complex)),
                 lambda: mn.nufft3d3(*x, c, *x),
                 lambda: mn.Type1PlanND(tuple(x), (8, 8, 8)),
                 lambda: mn.expi(np.zeros(4))):
        with pytest.raises(RuntimeError, match="GPU"):
            call()


def test_product_does_not_import_oracle():
    for f in (ROOT / "mlx_nufft_amd").rglob("*.py"):
        text = f.read_text()
        assert not re.search(r"^\s*(from|import)\s+oracle\b", text, re.M), f
        assert "liboracle" not in text, f


def test_bench_refuses_more_than_one_gpu():
    """bench.py runs on one GPU only: --gpus above 1 exits with status 2 and
    says so, before touching any device."""
    import subprocess
    import sys
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout.strip() == ""
