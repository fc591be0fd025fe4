"""The 3D type-1 hot path driven through the bare C-ABI, the way a reference
maintainer would bind it: a fresh ctypes.CDLL with its own signature table
(not the package's binding), device memory from torch, and only the calls
that replace Type1PlanND.execute and its point setup
(ref: mlx_nufft/nd.py:581-626, nd.py:152-372). The result must meet the
north-star gate against the exact direct sum:
    rel_l2(GPU, direct) <= max(eps, 2 * ref_err),
ref_err being the oracle's fp64 pipeline at the same (w, beta, n_up).
"""

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

c_i32, c_i64, c_f32, c_vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p
VP3, I64x3 = c_vp * 3, c_i64 * 3


class Bins(ctypes.Structure):
    _fields_ = [("dim", c_i32), ("w", c_i32), ("n", c_i64 * 3),
                ("m", c_i32 * 3), ("nb", c_i32 * 3)]


PB = ctypes.POINTER(Bins)
SIGS = [
    ("mn_last_error", ctypes.c_char_p, []),
    ("mn_zsweep_nkeys", c_i64, [PB]),
    ("mn_zsweep_setpts", c_i32, [PB, c_i64, VP3, c_i32, c_vp, VP3, c_vp]),
    ("mn_sort_pairs_workspace_bytes", c_i64, [c_i64, c_i32]),
    ("mn_sort_pairs", c_i32, [c_i64, c_i32, c_vp, c_vp, c_vp, c_i32, ctypes.POINTER(c_vp),
                              ctypes.POINTER(c_vp), c_vp, c_i64, c_vp]),
    ("mn_zsweep_starts", c_i32, [PB, c_i64, c_vp, c_vp, c_vp]),
    ("mn_spread_zsweep", c_i32, [PB, c_f32, c_i64, c_i32, c_vp, c_vp, c_vp, VP3, c_vp, c_vp,
                                 c_vp, c_vp]),
    ("mn_fftp_work_bytes", c_i64, [c_i32, I64x3, I64x3, c_i64]),
    ("mn_fft_crop_deconv", c_i32, [c_i32, I64x3, I64x3, c_i64, c_i32, c_vp, VP3, c_vp, c_i64,
                                   c_vp, c_vp]),
]


@pytest.fixture(scope="module")
def raw():
    from mlx_nufft_amd import _lib

    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    for name, res, args in SIGS:
        f = getattr(lib, name)
        f.restype, f.argtypes = res, args
    return lib


def _type1_raw(lib, x, c, N, w, beta, n_up, dec, isign):
    def check(rc, what):
        assert rc == 0, f"{what}: {lib.mn_last_error().decode()}"

    P = x[0].numel()
    s = c_vp(torch.cuda.current_stream().cuda_stream)
    g = Bins(dim=3, w=w)
    g.n[:] = n_up
    ptr = lambda t: c_vp(t.data_ptr())  # noqa: E731
    p3 = lambda ts: VP3(*[t.data_ptr() for t in ts])  # noqa: E731

    word = torch.empty(P, dtype=torch.int32, device="cuda")
    fr = torch.empty(3, P, dtype=torch.float32, device="cuda")
    check(lib.mn_zsweep_setpts(ctypes.byref(g), P, p3(x), 1, ptr(word), p3(fr), s), "setpts")
    K = lib.mn_zsweep_nkeys(ctypes.byref(g))
    ws = torch.empty(lib.mn_sort_pairs_workspace_bytes(P, 3), dtype=torch.uint8, device="cuda")
    sword, perm, frs = torch.empty_like(word), torch.empty_like(word), torch.empty_like(fr)
    cin = (c_vp * 3)(*[r.data_ptr() for r in fr])
    cout = (c_vp * 3)(*[r.data_ptr() for r in frs])
    check(lib.mn_sort_pairs(P, (K - 1).bit_length(), ptr(word), ptr(sword), ptr(perm), 3, cin,
                            cout, ptr(ws), ws.numel(), s), "sort")
    zstart = torch.empty(K + 1, dtype=torch.int32, device="cuda")
    check(lib.mn_zsweep_starts(ctypes.byref(g), P, ptr(sword), ptr(zstart), s), "starts")

    grid = torch.empty(int(np.prod(n_up)), dtype=torch.complex64, device="cuda")
    check(lib.mn_spread_zsweep(ctypes.byref(g), beta, P, 128, ptr(zstart), ptr(perm), ptr(sword),
                               p3(frs), ptr(c), None, ptr(grid), s), "spread")
    nu, NN = I64x3(*n_up), I64x3(*N)
    work = torch.empty(lib.mn_fftp_work_bytes(3, nu, NN, 1), dtype=torch.uint8, device="cuda")
    fk = torch.empty(N, dtype=torch.complex64, device="cuda")
    check(lib.mn_fft_crop_deconv(3, nu, NN, 1, isign, ptr(grid), p3(dec), ptr(work), work.numel(),
                                 ptr(fk), s), "fft")
    torch.cuda.synchronize()
    return fk.cpu().numpy()


@pytest.mark.parametrize("isign", [+1, -1])
def test_type1_through_bare_cabi(raw, oracle, isign):
    N, eps, M = (32, 16, 32), 1e-5, 30_000
    w, beta, n_up = oracle.type12_grid(N, eps)
    assert all(n % 8 == 0 for n in n_up[:2]) and all(n & (n - 1) == 0 for n in n_up)
    print(f"case bare-cabi t1 N={N} n_up={n_up} isign={isign}", flush=True)
    rng = np.random.default_rng(11)
    x = [rng.uniform(-np.pi, np.pi, M) for _ in range(3)]
    c = (rng.standard_normal(M) + 1j * rng.standard_normal(M)).astype(np.complex64)
    dec = [torch.from_numpy(v.astype(np.float32)).cuda() for v in oracle._decs(N, n_up, beta, w)]
    xd = [torch.from_numpy(v).cuda() for v in x]
    f = _type1_raw(raw, xd, torch.from_numpy(c).cuda(), N, w, beta, tuple(n_up), dec, isign)
    modes = [np.arange(-(n // 2), n - n // 2) for n in N]
    fe = oracle.dft_t1(x, c, modes, isign)
    ref_err = oracle.rel_l2(oracle.nufft_t1(x, c, N, eps, isign), fe)
    err = oracle.rel_l2(f, fe)
    print(f"  err={err:.3e} ref_err={ref_err:.3e}")
    assert err <= max(eps, 2 * ref_err)
