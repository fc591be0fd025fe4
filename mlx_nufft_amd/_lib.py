"""ctypes binding of the HIP C-ABI (include/mlx_nufft_amd.h) and the device
plumbing the plan classes share: torch tensors own all device memory, every
call runs on torch's current stream, and a non-zero status maps to the
Python exception class of the reference's error paths (ValueError,
RuntimeError, NotImplementedError).

There is no CPU fallback: without a ROCm GPU or without the built library
every entry point raises RuntimeError.
"""

import ctypes
import pathlib

import numpy as np
import torch

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libmlxnufft_amd.so"

c_int, c_int32, c_int64, c_float = ctypes.c_int, ctypes.c_int32, ctypes.c_int64, ctypes.c_float
c_vp = ctypes.c_void_p
VP3 = c_vp * 3
D3 = ctypes.c_double * 3
I64x3 = c_int64 * 3


class Bins(ctypes.Structure):
    """mn_bins: fine-grid bin geometry (see the C header)."""

    _fields_ = [("dim", c_int32), ("w", c_int32), ("n", c_int64 * 3),
                ("m", c_int32 * 3), ("nb", c_int32 * 3)]

    @classmethod
    def make(cls, dim, w, n, m):
        b = cls()
        b.dim, b.w = int(dim), int(w)
        for d in range(3):
            used = d < dim
            b.n[d] = int(n[d]) if used else 1
            b.m[d] = int(m[d]) if used else 1
            b.nb[d] = -(-int(n[d]) // int(m[d])) if used else 1
        return b

    @property
    def nbins(self):
        t = 1
        for d in range(self.dim):
            t *= self.nb[d]
        return t


# (name, restype, argtypes)
_SIGS = [
    ("mn_last_error", ctypes.c_char_p, []),
    ("mn_version", c_int, []),
    ("mn_device_lds_bytes", c_int, []),
    ("mn_setpts_t12", c_int, [ctypes.POINTER(Bins), c_int64, VP3, c_int, VP3, VP3, c_vp, c_vp]),
    ("mn_sort_workspace_bytes", c_int64, [c_int64]),
    ("mn_sort_keys", c_int, [c_int64, c_int, c_vp, c_vp, c_vp, c_vp, c_int64, c_vp]),
    ("mn_sort_pairs_workspace_bytes", c_int64, [c_int64, c_int]),
    ("mn_sort_pairs", c_int, [c_int64, c_int, c_vp, c_vp, c_vp, c_int, ctypes.POINTER(c_vp),
                              ctypes.POINTER(c_vp), c_vp, c_int64, c_vp]),
    ("mn_sort_pairs_noalloc", c_int, [c_int64, c_int, c_vp, c_vp, c_vp, c_int,
                                      ctypes.POINTER(c_vp), ctypes.POINTER(c_vp), c_vp]),
    ("mn_gather_points", c_int, [c_int, c_int64, c_vp, VP3, VP3, VP3, VP3, c_vp, c_vp, c_vp]),
    ("mn_subproblem_workspace_bytes", c_int64, [ctypes.POINTER(Bins)]),
    ("mn_build_subproblems", c_int, [ctypes.POINTER(Bins), c_int64, c_vp, c_int32, c_vp,
                                     c_int64, ctypes.POINTER(c_int64), c_vp, c_int64, c_vp]),
    ("mn_spread", c_int, [ctypes.POINTER(Bins), c_float, c_int64, c_int64, c_vp, c_vp, VP3, VP3,
                          c_vp, c_vp, c_vp, c_vp]),
    ("mn_spread_accumulate", c_int, [ctypes.POINTER(Bins), c_float, c_int64, c_int64, c_vp, c_vp,
                                     VP3, VP3, c_vp, c_vp, c_vp, c_vp]),
    ("mn_spread_c128", c_int, [ctypes.POINTER(Bins), c_float, c_int64, c_int64, c_vp, c_vp, VP3,
                               VP3, c_vp, c_vp, c_vp, c_vp]),
    ("mn_spread_owner_c128", c_int, [ctypes.POINTER(Bins), c_float, c_int64, c_vp, c_vp, VP3, VP3,
                                     c_vp, c_vp, c_vp, c_vp]),
    ("mn_zsweep_nkeys", c_int64, [ctypes.POINTER(Bins)]),
    ("mn_zsweep_setpts", c_int, [ctypes.POINTER(Bins), c_int64, VP3, c_int, c_vp, VP3, c_vp]),
    ("mn_zsweep_starts", c_int, [ctypes.POINTER(Bins), c_int64, c_vp, c_vp, c_vp]),
    ("mn_spread_zsweep", c_int, [ctypes.POINTER(Bins), c_float, c_int64, c_int, c_vp, c_vp, c_vp,
                                 VP3, c_vp, c_vp, c_vp, c_vp]),
    ("mn_spread_zsweep_batch", c_int, [ctypes.POINTER(Bins), c_float, c_int64, c_int64, c_int,
                                       c_vp, c_vp, c_vp, VP3, c_vp, c_vp, c_vp]),
    ("mn_zgather_setpts", c_int, [ctypes.POINTER(Bins), c_int64, VP3, c_int, c_vp, VP3, c_vp]),
    ("mn_interp_zgather", c_int, [ctypes.POINTER(Bins), c_float, c_int64, c_int64, c_int, c_vp,
                                  c_vp, c_vp, VP3, c_vp, c_vp, c_vp]),
    ("mn_permute_c64", c_int, [c_int64, c_vp, c_vp, c_vp, c_vp]),
    ("mn_pointmajor_c64", c_int, [c_int64, c_int64, c_vp, c_vp, c_vp]),
    ("mn_ysweep_nkeys", c_int64, [ctypes.POINTER(Bins)]),
    ("mn_ysweep_setpts", c_int, [ctypes.POINTER(Bins), c_int64, ctypes.c_void_p * 2, c_int, c_vp,
                                 ctypes.c_void_p * 2, c_vp]),
    ("mn_ysweep_starts", c_int, [ctypes.POINTER(Bins), c_int64, c_vp, c_vp, c_vp]),
    ("mn_spread_ysweep", c_int, [ctypes.POINTER(Bins), c_float, c_int64, c_int64, c_int, c_vp,
                                 c_vp, c_vp, ctypes.c_void_p * 2, c_vp, c_vp, c_vp]),
    ("mn_ymfma_nkeys", c_int64, [ctypes.POINTER(Bins)]),
    ("mn_ymfma_setpts", c_int, [ctypes.POINTER(Bins), c_int64, ctypes.c_void_p * 2, c_int, c_vp,
                                ctypes.c_void_p * 2, c_vp]),
    ("mn_ymfma_starts", c_int, [ctypes.POINTER(Bins), c_int64, c_vp, c_vp, c_vp]),
    ("mn_spread_ymfma", c_int, [ctypes.POINTER(Bins), c_float, c_int64, c_int64, c_int, c_vp,
                                c_vp, c_vp, ctypes.c_void_p * 2, c_vp, c_int, c_vp, c_vp]),
    ("mn_spread_batch", c_int, [ctypes.POINTER(Bins), c_float, c_int64, c_int64, c_vp, c_vp, VP3,
                                VP3, c_int64, c_vp, c_vp, c_vp]),
    ("mn_interp", c_int, [ctypes.POINTER(Bins), c_float, c_int64, c_int64, c_vp, c_vp, VP3, VP3,
                          c_vp, c_vp, c_vp, c_vp]),
    ("mn_bin_starts", c_int, [ctypes.POINTER(Bins), c_int64, c_vp, c_vp, c_vp]),
    ("mn_interp_direct", c_int, [ctypes.POINTER(Bins), c_float, c_int64, c_vp, VP3, VP3, c_vp, c_vp,
                                 c_vp, c_vp]),
    ("mn_interp_zstream", c_int, [ctypes.POINTER(Bins), c_float, c_int64, c_vp, c_vp, VP3, VP3,
                                  c_vp, c_vp, c_vp, c_vp]),
    ("mn_crop_deconv", c_int, [c_int, I64x3, I64x3, c_int64, c_vp, VP3, c_vp, c_vp]),
    ("mn_pad_deconv", c_int, [c_int, I64x3, I64x3, c_int64, c_vp, VP3, c_vp, c_vp]),
    ("mn_t3_setpts_src", c_int, [ctypes.POINTER(Bins), c_int64, VP3, D3, D3, D3, D3, c_int, c_int,
                                 VP3, VP3, c_vp, c_vp, c_vp]),
    ("mn_t3_setpts_trg", c_int, [ctypes.POINTER(Bins), c_int64, VP3, D3, D3, D3, D3, c_int, c_int,
                                 c_vp, c_int, VP3, VP3, c_vp, c_vp, c_vp]),
    ("mn_expi", c_int, [c_int, ctypes.POINTER(c_vp), c_int64, c_int, c_vp, c_vp]),
    ("mn_fft_exec", c_int, [c_int, I64x3, c_int64, c_int, c_vp, c_vp]),
    ("mn_fft_cache_clear", c_int, []),
    ("mn_fft_exec_f64", c_int, [c_int, I64x3, c_int64, c_int, c_vp, c_vp]),
    ("mn_pad_deconv_c128", c_int, [c_int, I64x3, I64x3, c_int64, c_vp, VP3, c_vp, c_vp]),
    ("mn_round_c64", c_int, [c_int64, c_vp, c_vp, c_vp]),
    ("mn_fft64_lines_supported", c_int, [c_int64]),
    ("mn_fft64_lines", c_int, [c_int64, c_int64, c_int64, c_int64, c_int, c_vp, c_vp, c_vp, c_int,
                               c_int, c_vp]),
    ("mn_transpose_c128", c_int, [c_int64, c_int64, c_int64, c_vp, c_vp, c_vp]),
    ("mn_fftp_supported", c_int, [c_int, I64x3]),
    ("mn_fftp_work_bytes", c_int64, [c_int, I64x3, I64x3, c_int64]),
    ("mn_fft_crop_deconv", c_int, [c_int, I64x3, I64x3, c_int64, c_int, c_vp, VP3, c_vp, c_int64,
                                   c_vp, c_vp]),
    ("mn_pad_deconv_fft", c_int, [c_int, I64x3, I64x3, c_int64, c_int, c_vp, VP3, c_vp, c_int64,
                                  c_vp, c_vp]),
    ("mn_fill_zero", c_int, [c_vp, c_int64, c_vp]),
]

EXPORTED = tuple(name for name, _, _ in _SIGS)

_lib = None


def load_library(path=None):
    """dlopen the C-ABI library and declare its signatures (no GPU needed)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = pathlib.Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise RuntimeError(
            f"mlx_nufft_amd: HIP library {p} is not built; run "
            "`python -m mlx_nufft_amd.build` (or __graft_entry__.build())")
    lib = ctypes.CDLL(str(p))
    for name, res, args in _SIGS:
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    if path is None:
        _lib = lib
    return lib


def lib():
    return load_library()


def require_gpu():
    """Fail loudly when no ROCm device is present: there is no CPU path."""
    if not torch.cuda.is_available():
        raise RuntimeError("mlx_nufft_amd requires a ROCm GPU (torch.cuda.is_available() is "
                           "False); there is no CPU fallback")
    return torch.device("cuda", torch.cuda.current_device())


_EXC = {-1: ValueError, -2: RuntimeError, -3: NotImplementedError}


def check(rc, what):
    if rc != 0:
        msg = lib().mn_last_error().decode(errors="replace")
        raise _EXC.get(rc, RuntimeError)(f"{what}: {msg}")


def require(cond, msg):
    """Raise ValueError(msg) unless cond. Used before raw device pointers go
    to the C side, which cannot see tensor sizes; unlike assert it is not
    stripped under python -O."""
    if not cond:
        raise ValueError(msg)


def stream():
    return c_vp(torch.cuda.current_stream().cuda_stream)


def ptr(t):
    return None if t is None else c_vp(t.data_ptr())


def ptr3(ts):
    ts = list(ts) + [None] * (3 - len(ts))
    return VP3(*[None if t is None else t.data_ptr() for t in ts])


def i64x3(vals):
    v = [int(x) for x in vals] + [1] * (3 - len(vals))
    return I64x3(*v)


def d3(vals):
    v = [float(x) for x in vals] + [0.0] * (3 - len(vals))
    return D3(*v)


# ---- host <-> device conversion ------------------------------------------

def is_device_tensor(a):
    return isinstance(a, torch.Tensor) and a.is_cuda


def to_dev_f64(a, dev):
    """1-D contiguous fp64 device copy (device fp64 tensors are used in place)."""
    if isinstance(a, torch.Tensor):
        t = a.detach().reshape(-1)
        if t.dtype != torch.float64 or t.device != dev:
            t = t.to(device=dev, dtype=torch.float64)
        return t.contiguous()
    arr = np.ascontiguousarray(np.asarray(a, dtype=np.float64).ravel())
    return torch.from_numpy(arr).to(dev)


def to_dev_c64(a, dev):
    """Contiguous complex64 device tensor (device complex64 tensors in place)."""
    if isinstance(a, torch.Tensor):
        t = a.detach()
        if t.dtype != torch.complex64 or t.device != dev:
            t = t.to(device=dev, dtype=torch.complex64)
        return t.contiguous()
    arr = np.ascontiguousarray(np.asarray(a).astype(np.complex64, copy=False))
    return torch.from_numpy(arr).to(dev)


def to_host(t):
    return t.cpu().numpy()
