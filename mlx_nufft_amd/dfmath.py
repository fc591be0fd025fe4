"""expi: e^{i*isign*phi} on the GPU for large-magnitude fp64 phases.

The reference forms the phase in double-single (df64) arithmetic and reduces
it mod 2pi before an fp32 cos/sin (ref: mlx_nufft/dfmath.py:1-134). CDNA4
has native fp64, so here the components are summed in fp64 and the fp64
sincos reduces and evaluates the phase; the complex64 result has no
magnitude ceiling. EXPI_MAX_PHASE is kept for API compatibility: it is the
reference's df64 validity bound (|phi| for which phi/2pi stays an exact
fp32 integer), below which both implementations agree to ~1e-7.
"""

import numpy as np
import torch

from . import _engine as E
from . import _lib as L

PI = np.pi

EXPI_MAX_PHASE = float(2 ** 24 * 2.0 * PI)


def expi(phases, isign=1, return_np=False):
    """e^{i*isign*phi} as complex64, same shape as the input.

    phases: an fp64 array (numpy or torch), or a sequence of same-shape
    arrays that are summed (in fp64, on the GPU) to form phi. A flat
    list/tuple of scalars is rejected (it would be summed into one phase).
    isign: normalised by sign (>= 0 -> +1). return_np: numpy result instead
    of the device tensor. NaN/inf phases give NaN per element.
    ref: dfmath.py:57-134.
    """
    if isinstance(phases, (list, tuple)):
        comps = list(phases)
    else:
        comps = [phases]
    if len(comps) < 1:
        raise ValueError("expi: at least one phase component is required")
    if len(comps) > 8:
        raise ValueError("expi: at most 8 phase components are supported")
    shapes = [tuple(c.shape) if isinstance(c, torch.Tensor) else np.shape(c) for c in comps]
    shape = shapes[0]
    if any(sh != shape for sh in shapes):
        raise ValueError("expi: all phase components must share one shape")
    if len(comps) > 1 and shape == ():
        raise ValueError(
            "expi: got a multi-element sequence of scalars, which would be summed into a "
            "single phase. Pass np.asarray(...) for a vector of per-element phases, or 1-D "
            "arrays as summable phase components.")
    isign = +1 if isign >= 0 else -1
    dev = L.require_gpu()
    dc = [L.to_dev_f64(c, dev) for c in comps]
    out = torch.empty(shape, dtype=torch.complex64, device=dev)
    if out.numel():
        E.expi(dc, isign, out)
    return L.to_host(out) if return_np else out
