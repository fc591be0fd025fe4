"""Legacy 3D-only type-1/2 plans, kept for API compatibility.

The reference's Type1Plan/Type2Plan (ref: mlx_nufft/types12.py:94-290) are
3D, even-N plans with sigma=1.25 and eps=1e-5 defaults whose kernels were
superseded by the ND engine; here they are thin subclasses of the ND plans
with those defaults.
"""

import numpy as np

from .nd import Type1PlanND, Type2PlanND


def _check3(x, n_modes):
    if len(tuple(x)) != 3:
        raise ValueError("Type1Plan/Type2Plan are 3D plans (3 coordinate arrays)")
    N = (int(n_modes),) * 3 if np.isscalar(n_modes) else tuple(int(n) for n in n_modes)
    if len(N) != 3:
        raise ValueError("n_modes must have 3 entries")
    return tuple(x), N


class Type1Plan(Type1PlanND):
    """3D type 1, f[k] = sum_j c[j] exp(i*isign k.x_j) (ref: types12.py:94-179)."""

    def __init__(self, x, n_modes, eps=1e-5, isign=+1, upsampfac=1.25, prec="crit64",
                 sort_points=True):
        x, N = _check3(x, n_modes)
        super().__init__(x, N, eps=eps, isign=isign, upsampfac=upsampfac, prec=prec,
                         sort_points=sort_points)


class Type2Plan(Type2PlanND):
    """3D type 2, c[j] = sum_k f[k] exp(i*isign k.x_j) (ref: types12.py:182-290)."""

    def __init__(self, x, n_modes, eps=1e-5, isign=-1, upsampfac=1.25, prec="crit64",
                 sort_points=True):
        x, N = _check3(x, n_modes)
        super().__init__(x, N, eps=eps, isign=isign, upsampfac=upsampfac, prec=prec,
                         sort_points=sort_points)
