"""The XCD-grouped block order of the larger-M quant GEMM (qgemm.hip,
qgemm_rows with KParams.swz != 0) must visit every (column block, row block)
tile exactly once, leave only padding blocks without a tile, and give each
XCD (block id mod 8) only blocks of its own residue in the owned dimension
(columns for swz > 0, rows for swz < 0).  The order is restated here from
the kernel's prologue and checked as a bijection over a range of grid shapes
and group sizes, padded ones included."""
import itertools


def tile_of(b, nbx, nby, swz):
    cols = swz > 0
    own, other = (nbx, nby) if cols else (nby, nbx)
    x, local, per = b & 7, b >> 3, (own + 7) >> 3
    G = min(abs(swz), per)
    gi = local // (G * other)
    r = local - gi * G * other
    Gg = min(G, per - gi * G)
    o = r // Gg
    w = x + 8 * (gi * G + (r - o * Gg))
    bx, by = (w, o) if cols else (o, w)
    return None if bx >= nbx or by >= nby else (bx, by)


def grid_of(nbx, nby, swz):
    return (nbx + 7) // 8 * 8 * nby if swz > 0 else (nby + 7) // 8 * 8 * nbx


def test_grouped_order_is_a_bijection_and_xcd_local():
    for nbx, nby, g in itertools.product((3, 8, 13, 16, 20, 28, 80, 136), (2, 3, 17, 34, 68), (1, 2, 3, 5, 8, 40)):
        for swz in (g, -g):
            seen = set()
            for b in range(grid_of(nbx, nby, swz)):
                t = tile_of(b, nbx, nby, swz)
                if t is None:
                    continue
                bx, by = t
                assert 0 <= bx < nbx and 0 <= by < nby
                assert (bx if swz > 0 else by) % 8 == b % 8
                assert t not in seen
                seen.add(t)
            assert len(seen) == nbx * nby, (nbx, nby, swz)
