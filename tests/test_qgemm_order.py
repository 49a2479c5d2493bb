"""The XCD-grouped block order of the larger-M quant GEMM (qgemm.hip,
qgemm_rows with KParams.swz > 0) must visit every (column block, row block)
tile exactly once, and give each XCD (block id mod 8) only column blocks of
its own residue.  The order is restated here from the kernel's prologue and
checked as a bijection over a range of grid shapes and group sizes."""
import itertools


def tile_of(b, nbx, nby, swz):
    x, local, per = b & 7, b >> 3, nbx >> 3
    G = min(swz, per)
    gi = local // (G * nby)
    r = local - gi * G * nby
    Gg = min(G, per - gi * G)
    by = r // Gg
    bx = x + 8 * (gi * G + (r - by * Gg))
    return bx, by


def test_grouped_order_is_a_bijection_and_xcd_local():
    for nbx, nby, swz in itertools.product((8, 16, 24, 80, 136), (2, 3, 17, 68), (1, 2, 3, 5, 8, 40)):
        seen = set()
        for b in range(nbx * nby):
            bx, by = tile_of(b, nbx, nby, swz)
            assert 0 <= bx < nbx and 0 <= by < nby
            assert bx % 8 == b % 8
            seen.add((bx, by))
        assert len(seen) == nbx * nby, (nbx, nby, swz)
