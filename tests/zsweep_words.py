"""The z-sweep point word restated in numpy (shared by the host and GPU tests).

ref: nd.py:152-165 (cells); the word layout is this engine's own (the
owner-computes spread's sort key).
"""

import numpy as np


def reach(o, w):
    """Reach code of a first tap at cell o of its 8-column block: 0 stays in
    the block; else 1 also covers the block's lower half (o <= 3), 3 also
    the next block's upper half (o + w - 1 >= 12), 2 neither."""
    return np.where(o + w - 1 < 8, 0, np.where(o <= 3, 1, np.where(o + w - 1 >= 12, 3, 2)))


def rank(cx, cy):
    """Key rank of class (cx, cy): classes reaching along x take 3..14, along
    y 0..11, so each neighbour's reaching points are one key range."""
    return np.where(cx == 0, np.where(cy == 0, 15, cy - 1), np.where(cy == 0, 11 + cx,
                                                                     3 * cx + cy - 1))


def words_numpy(i1, n, w):
    """The z-sweep point word: key ((bx*nby + by)*nzc + z//8)*16 + rank in
    bits 0-22, the in-block x / y cell of the first tap in bits 23-25 /
    26-28, its cell in its 8-cell z-chunk in bits 29-31."""
    x, y, z = (i1[d].astype(np.int64) % n[d] for d in range(3))
    nzc = -(-n[2] // 8)
    blk = (x // 8) * (n[1] // 8) + y // 8
    key = (blk * nzc + z // 8) * 16 + rank(reach(x % 8, w), reach(y % 8, w))
    word = key | ((x % 8) << 23) | ((y % 8) << 26) | ((z % 8) << 29)
    return key.astype(np.uint32), word.astype(np.uint32), (n[0] // 8) * (n[1] // 8) * nzc * 16
