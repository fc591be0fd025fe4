"""mlx_nufft_amd: non-uniform FFTs (types 1, 2, 3 in 1D/2D/3D) on AMD
Instinct MI355X (gfx950), with the finufft-compatible surface of mlx-nufft.

    import mlx_nufft_amd as finufft
    fk = finufft.nufft2d1(x, y, c, (N1, N2), eps=1e-6)
    plan = finufft.Plan(1, (N1, N2), eps=1e-6)
    plan.setpts(x, y)
    fk = plan.execute(c)

plus the native plan classes (Type1PlanND, Type2PlanND, Type3Plan) and
expi. Precision model: fp32 execute pipeline with the precision-critical
setup (coordinate fold/rescale, phases) in native fp64 on the GPU ("crit64").
Device work runs in hand-written HIP kernels behind a C-ABI
(include/mlx_nufft_amd.h, libmlxnufft_amd.so) plus rocFFT; torch tensors
hold the device buffers. ref: mlx_nufft/__init__.py:1-48.
"""

from .api import (Plan, nufft1d1, nufft1d2, nufft1d3, nufft2d1, nufft2d2, nufft2d3,
                  nufft3d1, nufft3d2, nufft3d3)
from .dfmath import EXPI_MAX_PHASE, expi
from .nd import Type1PlanND, Type2PlanND
from .sizing import kernel_params, next235even
from .t3 import GpuT3Plan as Type3Plan
from .types12 import Type1Plan, Type2Plan


def vkfft_available():
    """The reference's optional VkFFT-Metal backend does not exist on this
    platform (rocFFT is built in), so this is always False."""
    return False


__version__ = "0.1.3"
__all__ = ["Type3Plan", "Type1Plan", "Type2Plan",
           "Type1PlanND", "Type2PlanND", "Plan",
           "nufft1d1", "nufft1d2", "nufft1d3",
           "nufft2d1", "nufft2d2", "nufft2d3",
           "nufft3d1", "nufft3d2", "nufft3d3",
           "kernel_params", "next235even", "vkfft_available",
           "expi", "EXPI_MAX_PHASE"]
