"""Write tests/golden/fullsize_ref.json: the CPU oracle's own error at each
BASELINE configuration's full size, on the samples tests/fullsize_cases.py
fixes. The GPU gate is rel_l2(GPU, direct) <= max(eps, 2 * ref_err); at these
sizes the fp64 oracle takes minutes (a 3D spread of 2e7 points alone is
about a minute on 8 cores), so its error is computed once here, on the CPU,
and committed. The direct sums on the samples are cheap and are recomputed
by the GPU tests themselves.

    python tests/golden/make_fullsize_ref.py      # a few minutes, ~8 GB RAM
"""

import json
import pathlib
import sys
import time

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

import fullsize_cases as F  # noqa: E402
from oracle import oracle as O  # noqa: E402


def sub_modes(full, N, modes):
    """Values of a modeord-0 mode array at the tensor sub-grid `modes`."""
    idx = np.ix_(*[np.asarray(m) + n // 2 for m, n in zip(modes, N)])
    return full[idx]


def main(only=None):
    """only: a set of case names to recompute; the others keep their
    committed values."""
    O.lib()
    path = HERE / "fullsize_ref.json"
    out = json.loads(path.read_text()) if only and path.exists() else {}
    t0 = time.time()

    if not only or "cfg0_1d_t1" in only:
        k = F.cfg0_1d_t1()
        fe = O.dft_t1(k["x"], k["c"], k["modes"], k["isign"])
        fo = O.nufft_t1(k["x"], k["c"], k["N"], k["eps"], k["isign"])
        out["cfg0_1d_t1"] = {"eps": k["eps"], "ref_err": O.rel_l2(fo, fe)}
        print("cfg0", out["cfg0_1d_t1"], f"{time.time() - t0:.0f}s", flush=True)

    if not only or "cfg1_2d_t1_batched" in only:
        k = F.cfg1_2d_t1_batched()
        errs = {}
        for b in k["checked"]:
            fe = O.dft_t1(k["x"], k["cs"][b], k["modes"], k["isign"])
            fo = O.nufft_t1(k["x"], k["cs"][b], k["N"], k["eps"], k["isign"])
            errs[str(b)] = O.rel_l2(sub_modes(fo, k["N"], k["modes"]), fe)
        out["cfg1_2d_t1_batched"] = {"eps": k["eps"], "ref_err": errs}
        print("cfg1", out["cfg1_2d_t1_batched"], f"{time.time() - t0:.0f}s", flush=True)

    if not only or "cfg2_2d_t2_radial" in only:
        k = F.cfg2_2d_t2_radial()
        ce = O.dft_t2(k["x"], k["f"], k["isign"], k["points"])
        co = O.nufft_t2(k["x"], k["f"], k["eps"], k["isign"])[k["points"]]
        out["cfg2_2d_t2_radial"] = {"eps": k["eps"], "ref_err": O.rel_l2(co, ce)}
        print("cfg2", out["cfg2_2d_t2_radial"], f"{time.time() - t0:.0f}s", flush=True)

    if not only or "cfg3_3d_t1" in only:
        k = F.cfg3_3d_t1()
        fe = O.dft_t1(k["x"], k["c"], k["modes"], k["isign"])
        fo = O.nufft_t1(k["x"], k["c"], k["N"], k["eps"], k["isign"])
        out["cfg3_3d_t1"] = {"eps": k["eps"],
                             "ref_err": O.rel_l2(sub_modes(fo, k["N"], k["modes"]), fe)}
        del fo
        print("cfg3", out["cfg3_3d_t1"], f"{time.time() - t0:.0f}s", flush=True)

    if not only or "cfg4_3d_t3" in only:
        k = F.cfg4_3d_t3()
        fe = O.dft_t3(k["x"], k["c"], k["s"], k["isign"], k["targets"])
        e64 = O.rel_l2(O.nufft_t3(k["x"], k["c"], k["s"], k["eps"], k["isign"])[k["targets"]], fe)
        e32 = O.rel_l2(O.nufft_t3(k["x"], k["c"], k["s"], k["eps"], k["isign"],
                                  spread64=False)[k["targets"]], fe)
        out["cfg4_3d_t3"] = {"eps": k["eps"], "ref_err": max(e64, e32), "ref_err_fp64": e64,
                             "ref_err_fp32_spread": e32}
        print("cfg4", out["cfg4_3d_t3"], f"{time.time() - t0:.0f}s", flush=True)

    path.write_text(json.dumps(out, indent=1) + "\n")


if __name__ == "__main__":
    main(set(sys.argv[1:]) or None)
