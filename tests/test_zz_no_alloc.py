"""The no-allocation sort entry point, mn_sort_pairs_noalloc, called through
the C-ABI: its workspace is the library's device scratch array instead of a
caller buffer. It must give exactly what mn_sort_pairs gives with a
workspace (keys, permutation and payload columns bit for bit, the
permutation being numpy's stable argsort), on two calls in a row with the
second smaller (the scratch keeps the first call's contents), and it must
refuse a sort whose workspace exceeds the scratch array before any device
work.
"""

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 96 << 20


def _sort(lib, L, P, bits, key, cols, noalloc):
    dev = key.device
    kout = torch.empty_like(key)
    perm = torch.empty_like(key)
    outs = [torch.empty_like(c) for c in cols]
    VP = ctypes.c_void_p
    cin = (VP * max(1, len(cols)))(*[c.data_ptr() for c in cols])
    cout = (VP * max(1, len(cols)))(*[c.data_ptr() for c in outs])
    if noalloc:
        rc = lib.mn_sort_pairs_noalloc(P, bits, L.ptr(key), L.ptr(kout), L.ptr(perm), len(cols),
                                       cin, cout, L.stream())
    else:
        nbytes = int(lib.mn_sort_pairs_workspace_bytes(P, len(cols)))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        rc = lib.mn_sort_pairs(P, bits, L.ptr(key), L.ptr(kout), L.ptr(perm), len(cols), cin,
                               cout, L.ptr(ws), nbytes, L.stream())
    L.check(rc, "noalloc" if noalloc else "sort")
    torch.cuda.synchronize()
    return kout.cpu().numpy(), perm.cpu().numpy(), [o.cpu().numpy() for o in outs]


def test_sort_pairs_noalloc_equals_workspace_sort():
    from mlx_nufft_amd import _lib as L

    lib = L.lib()
    dev = torch.device("cuda")
    # the second call is smaller than the first; the last case has no payload
    for P, ncols, bits, seed in ((4_000_000, 3, 23, 1), (250_001, 2, 17, 2), (9_000, 0, 32, 3)):
        print(f"case noalloc sort P={P} ncols={ncols} bits={bits}", flush=True)
        assert lib.mn_sort_pairs_workspace_bytes(P, ncols) <= SCRATCH_BYTES
        rng = np.random.default_rng(seed)
        keys = rng.integers(0, 2 ** 32, P, dtype=np.uint64).astype(np.uint32)
        keys[: P // 3] &= np.uint32(0xFF)          # many equal keys: stability matters
        key = torch.from_numpy(keys.view(np.int32)).to(dev)
        cols = [torch.from_numpy(rng.integers(-2 ** 31, 2 ** 31, P, dtype=np.int64)
                                 .astype(np.int32)).to(dev) for _ in range(ncols)]
        k1, p1, c1 = _sort(lib, L, P, bits, key, cols, noalloc=False)
        k2, p2, c2 = _sort(lib, L, P, bits, key, cols, noalloc=True)
        assert np.array_equal(k1, k2) and np.array_equal(p1, p2)
        for a, b in zip(c1, c2):
            assert np.array_equal(a, b)
        mask = np.uint32(0xFFFFFFFF) if bits == 32 else np.uint32((1 << bits) - 1)
        want = np.argsort(keys & mask, kind="stable")
        assert np.array_equal(p2.view(np.uint32).astype(np.int64), want)
        for c, out in zip(cols, c2):
            assert np.array_equal(out, c.cpu().numpy()[want])


def test_sort_pairs_noalloc_rejects_oversize():
    from mlx_nufft_amd import _lib as L

    lib = L.lib()
    P = 6_000_000   # with 3 payload columns this needs about 115 MiB
    assert lib.mn_sort_pairs_workspace_bytes(P, 3) > SCRATCH_BYTES
    t = torch.empty(16, dtype=torch.int32, device="cuda")
    VP = ctypes.c_void_p
    cols = (VP * 3)(*[t.data_ptr()] * 3)
    rc = lib.mn_sort_pairs_noalloc(P, 23, L.ptr(t), L.ptr(t), L.ptr(t), 3, cols, cols,
                                   L.stream())
    assert rc == -1
    assert "scratch" in lib.mn_last_error().decode()
