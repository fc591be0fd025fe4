"""The full-size reference-error fixture (tests/golden/fullsize_ref.json)
against the current oracle, on the one configuration cheap enough to
recompute on the CPU (1D, M = 1e5, N = 4096), and its shape for the rest."""

import json
import pathlib

import fullsize_cases as F

REF = json.loads((pathlib.Path(__file__).resolve().parent / "golden" / "fullsize_ref.json")
                 .read_text())


def test_fixture_matches_oracle_cfg0(oracle):
    k = F.cfg0_1d_t1()
    fe = oracle.dft_t1(k["x"], k["c"], k["modes"], k["isign"])
    fo = oracle.nufft_t1(k["x"], k["c"], k["N"], k["eps"], k["isign"])
    assert abs(oracle.rel_l2(fo, fe) - REF["cfg0_1d_t1"]["ref_err"]) <= 1e-9


def test_fixture_fields():
    assert set(REF) == {"cfg0_1d_t1", "cfg1_2d_t1_batched", "cfg2_2d_t2_radial", "cfg3_3d_t1",
                        "cfg4_3d_t3"}
    for case, r in REF.items():
        vals = r["ref_err"].values() if isinstance(r["ref_err"], dict) else [r["ref_err"]]
        # the fp64 oracle reaches eps-level at every configuration (at most
        # 5x eps: the type-3 value is the reference's fp32-spread stage)
        assert all(0 < v < 5 * r["eps"] for v in vals), case
