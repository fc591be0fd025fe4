"""Legacy 3D type-1/2 plans, kept for API compatibility.

The reference's Type1Plan/Type2Plan (ref: mlx_nufft/types12.py:94-290) are
3D plans on even mode boxes with eps=1e-5 and upsampfac=1.25 defaults; both
default to isign=+1, Type1Plan sorts its points and Type2Plan does not
(ref: types12.py:163-164, 185-186). Their kernels were superseded by the ND
engine, so here they are the ND plans with those defaults and with the
reference's checks: three coordinate arrays and three even mode sizes
(ref: types12.py:36-37). The checks raise PlanArgumentError, which is both
the ValueError an API user expects and the AssertionError the reference's
assert raises.
"""

import numpy as np

from .nd import PlanArgumentError, Type1PlanND, Type2PlanND


def _legacy_args(x, n_modes, prec):
    if prec not in ("fp32", "crit64"):
        raise PlanArgumentError(f"prec must be 'fp32' or 'crit64', got {prec!r}")
    coords = tuple(x)
    if len(coords) != 3:
        raise PlanArgumentError(f"legacy plans are 3D: they take 3 coordinate arrays, got "
                                f"{len(coords)}")
    box = (n_modes,) * 3 if np.isscalar(n_modes) else tuple(n_modes)
    box = tuple(int(n) for n in box)
    if len(box) != 3 or any(n % 2 for n in box):
        raise PlanArgumentError(f"legacy plans need 3 even mode sizes, got {box}")
    return coords, box


class Type1Plan(Type1PlanND):
    """3D type 1, f[k] = sum_j c[j] exp(i*isign k.x_j), on an even mode box
    (ref: types12.py:159-179)."""

    def __init__(self, x, n_modes, eps=1e-5, isign=+1, upsampfac=1.25, prec="crit64",
                 sort_points=True):
        coords, box = _legacy_args(x, n_modes, prec)
        super().__init__(coords, box, eps=eps, isign=isign, upsampfac=upsampfac, prec=prec,
                         sort_points=sort_points)


class Type2Plan(Type2PlanND):
    """3D type 2, c[j] = sum_k f[k] exp(i*isign k.x_j), on an even mode box
    (ref: types12.py:182-290). Results come back in caller point order."""

    def __init__(self, x, n_modes, eps=1e-5, isign=+1, upsampfac=1.25, prec="crit64",
                 sort_points=False):
        coords, box = _legacy_args(x, n_modes, prec)
        super().__init__(coords, box, eps=eps, isign=isign, upsampfac=upsampfac, prec=prec,
                         sort_points=sort_points)
