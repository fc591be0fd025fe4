"""GPU parity of plan-time point setup, the bin sort and the subproblem table.

Bar: bit-exact. i1 and fr against the CPU oracle (itself pinned to numpy's
np.mod/ceil in test_oracle.py), bin keys against the oracle's key function,
the permutation against numpy's argsort(kind="stable") on the same keys
(ref: nd.py:314), and the subproblem rows against a numpy restatement of
the reference's table build (ref: nd.py:347-360).
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

TWO_PI = 2.0 * np.pi


def _coords(rng, dim, P):
    """Half in [-pi, pi), half over +-1000*2pi, plus edge values."""
    edge = np.array([0.0, -0.0, TWO_PI, -TWO_PI, np.pi, -np.pi, 1e-300, -1e-300, -5e-324,
                     -1e-17, 1e-17, 7e15, -7e15, 3 * TWO_PI, -1000 * TWO_PI, 12345.678,
                     np.nextafter(TWO_PI, 0), np.nextafter(-np.pi, 0)])
    out = []
    for _ in range(dim):
        a = rng.uniform(-np.pi, np.pi, P // 2)
        b = rng.uniform(-1000 * TWO_PI, 1000 * TWO_PI, P - P // 2 - edge.size)
        out.append(np.concatenate([a, b, rng.permutation(edge)]))
    return out


@pytest.mark.parametrize("dim,N", [(1, (4096,)), (2, (2048, 2048)), (3, (256, 256, 128)),
                                   (3, (21, 18, 14))])
@pytest.mark.parametrize("prec", ["crit64", "fp32"])
def test_setpts_bitexact(dim, N, prec, oracle):
    from mlx_nufft_amd import _engine as E

    print(f"case setpts dim={dim} N={N} prec={prec}", flush=True)
    rng = np.random.default_rng(11)
    x = _coords(rng, dim, 60_000)
    w, beta, n_up = oracle.type12_grid(N, 1e-5)
    i1o, fro = oracle.setpts_t12(x, n_up, w, prec == "crit64")
    bins = E.make_bins(dim, w, n_up)
    xd = [torch.from_numpy(v).cuda() for v in x]
    i1, fr, key = E.setpts_t12(bins, xd, prec == "crit64")
    i1, fr, key = i1.cpu().numpy(), fr.cpu().numpy(), key.cpu().numpy().view(np.uint32)
    assert np.array_equal(i1, i1o), f"i1 mismatches: {np.sum(i1 != i1o)}"
    assert np.array_equal(fr.view(np.int32), fro.view(np.int32)), \
        f"fr mismatches: {np.sum(fr != fro)} max {np.max(np.abs(fr - fro))}"
    ko, _ = oracle.bin_keys(i1o, n_up, [bins.m[d] for d in range(dim)], w)
    assert np.array_equal(key, ko)


def _keys_for(oracle, x, N, eps=1e-5):
    from mlx_nufft_amd import _engine as E

    dim = len(x)
    w, beta, n_up = oracle.type12_grid(N, eps)
    bins = E.make_bins(dim, w, n_up)
    i1o, _ = oracle.setpts_t12(x, n_up, w)
    ko, nk = oracle.bin_keys(i1o, n_up, [bins.m[d] for d in range(dim)], w)
    return bins, ko, nk


@pytest.mark.parametrize("case", ["uniform3d_2M", "cluster3d", "uniform2d", "tiny1", "tile_edge",
                                  "all_equal"])
def test_sort_matches_numpy_stable(case, oracle):
    from mlx_nufft_amd import _engine as E

    print(f"case sort {case}", flush=True)
    rng = np.random.default_rng(5)
    if case == "uniform3d_2M":
        x, N = [rng.uniform(-np.pi, np.pi, 2_000_000) for _ in range(3)], (256,) * 3
    elif case == "cluster3d":
        h = 2 * np.pi / 512
        x, N = [-np.pi + rng.uniform(0, 8 * h, 300_000) for _ in range(3)], (256,) * 3
    elif case == "uniform2d":
        x, N = [rng.uniform(-np.pi, np.pi, 1_000_003) for _ in range(2)], (1024, 1024)
    elif case == "tiny1":
        x, N = [rng.uniform(-np.pi, np.pi, 1)], (64,)
    elif case == "tile_edge":
        x, N = [rng.uniform(-np.pi, np.pi, 4097) for _ in range(2)], (96, 80)
    else:
        x, N = [np.full(10_000, 0.5) for _ in range(3)], (32, 32, 32)
    bins, ko, nk = _keys_for(oracle, x, N)
    ref = np.argsort(ko, kind="stable")
    kd = torch.from_numpy(ko.view(np.int32)).cuda()
    skey, perm = E.sort_keys(kd, E.key_bits(bins))
    perm = perm.cpu().numpy().view(np.uint32)
    assert np.array_equal(perm, ref.astype(np.uint32))
    assert np.array_equal(skey.cpu().numpy().view(np.uint32), ko[ref])
    # the oracle's own counting sort agrees too
    assert np.array_equal(oracle.stable_sort(ko, nk), ref.astype(np.uint32))


@pytest.mark.parametrize("P,nbits,ncols", [(1, 5, 3), (4095, 7, 0), (4097, 12, 1),
                                             (300_001, 23, 3), (1_000_000, 32, 8),
                                             (65_536, 16, 6), (4096 * 8192 + 3, 22, 1),
                                             (50_001, 10, 2), (200_003, 17, 1),
                                             (100_000, 25, 0), (8192 * 3, 11, 3),
                                             (70_001, 9, 1), (1000, 0, 1)])
def test_sort_pairs_payload(P, nbits, ncols):
    """Stable sort on the low nbits of each key, bits above nbits travelling
    with the key, and payload columns following their keys: against numpy's
    stable argsort. Key widths from one pass (5, 7) to four (25, 32); the
    passes split the key evenly (9 bits as 5 + 4, 10 as 5 + 5, 17 as
    6 + 6 + 5, 22 as 8 + 7 + 7, 25 as 7 + 6 + 6 + 6); 0 bits leave the
    order unchanged. The 22-bit case has 4097 tiles of 8192
    keys, so the per-digit scan over the tiles runs its carry loop twice;
    the 11-bit case fills exactly three tiles."""
    from mlx_nufft_amd import _engine as E

    print(f"case sort_pairs P={P} nbits={nbits} ncols={ncols}", flush=True)
    rng = np.random.default_rng(P + nbits)
    key = rng.integers(0, 1 << 32, P, dtype=np.uint64).astype(np.uint32)
    low = key & np.uint32(0xFFFFFFFF if nbits == 32 else (1 << nbits) - 1)
    if nbits >= 12:   # many ties
        low[rng.integers(0, P, P // 3)] = low[0]
        key = (key & ~np.uint32((1 << nbits) - 1 if nbits < 32 else 0xFFFFFFFF)) | low
    cols = [rng.integers(-2**31, 2**31, P, dtype=np.int64).astype(np.int32) for _ in range(ncols)]
    ref = np.argsort(low, kind="stable")
    kd = torch.from_numpy(key.view(np.int32)).cuda()
    cd = [torch.from_numpy(c).cuda() for c in cols]
    skey, perm, outs = E.sort_pairs(kd, nbits, cd)
    assert np.array_equal(perm.cpu().numpy().view(np.uint32), ref.astype(np.uint32))
    assert np.array_equal(skey.cpu().numpy().view(np.uint32), key[ref])
    for c, o in zip(cols, outs):
        assert np.array_equal(o.cpu().numpy(), c[ref])


@pytest.mark.parametrize("offset", [1, 3])
def test_sort_pairs_misaligned_keys(offset):
    """Keys that start 4 or 12 bytes past a 16-byte boundary: the histogram
    pass reads whole tiles as 16-byte vectors only from aligned key arrays,
    and element by element otherwise. Five whole 8192-key tiles and a
    partial one, against numpy's stable argsort."""
    from mlx_nufft_amd import _engine as E

    P, nbits = 8192 * 5 + 17, 22
    print(f"case sort_pairs misaligned offset={offset}", flush=True)
    rng = np.random.default_rng(40 + offset)
    key = rng.integers(0, 1 << 32, P, dtype=np.uint64).astype(np.uint32)
    key[rng.integers(0, P, P // 4)] = key[0]   # ties
    col = rng.integers(-2**31, 2**31, P, dtype=np.int64).astype(np.int32)
    padded = np.concatenate([np.zeros(offset, np.uint32), key])
    kd = torch.from_numpy(padded.view(np.int32)).cuda()[offset:]
    assert kd.data_ptr() % 16 == 4 * offset
    skey, perm, outs = E.sort_pairs(kd, nbits, [torch.from_numpy(col).cuda()])
    ref = np.argsort(key & np.uint32((1 << nbits) - 1), kind="stable")
    assert np.array_equal(perm.cpu().numpy().view(np.uint32), ref.astype(np.uint32))
    assert np.array_equal(skey.cpu().numpy().view(np.uint32), key[ref])
    assert np.array_equal(outs[0].cpu().numpy(), col[ref])


@pytest.mark.parametrize("msub", [1024, 7])
def test_subproblem_table(msub, oracle):
    from mlx_nufft_amd import _engine as E

    print(f"case subproblems msub={msub}", flush=True)
    rng = np.random.default_rng(6)
    h = 2 * np.pi / 128
    x = [np.concatenate([rng.uniform(-np.pi, np.pi, 50_000), -np.pi + rng.uniform(0, 4 * h, 20_000)])
         for _ in range(3)]
    bins, ko, nk = _keys_for(oracle, x, (64, 64, 64))
    ks = np.sort(ko, kind="stable")
    info, nsub = E.build_subproblems(bins, torch.from_numpy(ks.view(np.int32)).cuda(), msub)
    info = info[:nsub].cpu().numpy()
    # numpy restatement of the reference's table build (nd.py:351-360)
    starts = np.flatnonzero(np.r_[True, ks[1:] != ks[:-1]])
    counts = np.diff(np.r_[starts, ks.size])
    per = (counts + msub - 1) // msub
    bin_id = np.repeat(np.arange(starts.size), per)
    seg = np.cumsum(per) - per
    off = (np.arange(per.sum()) - np.repeat(seg, per)) * msub
    exp = np.stack([ks[starts][bin_id].astype(np.int64), starts[bin_id] + off,
                    np.minimum(msub, counts[bin_id] - off)], axis=1)
    assert nsub == exp.shape[0]
    assert np.array_equal(info.astype(np.int64), exp)
