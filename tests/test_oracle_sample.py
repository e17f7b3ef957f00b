"""The spread sample checker (oracle/sample.py) and the strided generator it
regenerates operands with, pinned on the CPU: the sample covers every tile
row and tile column, agrees with a full FP64 check on a correct product, and
catches the mistakes the mod-3/mod-5 pattern cannot see (a C block routed to
the wrong place, a stale block, one wrong element)."""
import numpy as np
import pytest

import oracle
from oracle.sample import SeededOperand, spread_check, spread_positions


def test_strided_fill_matches_contiguous():
    full = oracle.fill_uniform(64 * 48, 7)
    stored = full.reshape(48, 64).T  # 64 x 48 column-major
    blk = oracle.fill_uniform_strided(5, 4, 7, 3 + 2 * 64, 1, 64)
    np.testing.assert_array_equal(blk, stored[3:8, 2:6])
    row = oracle.fill_uniform_strided(1, 48, 7, 10, 0, 64)
    np.testing.assert_array_equal(row[0], stored[10, :])


@pytest.mark.parametrize("transposed", [False, True])
def test_seeded_operand_views_agree(transposed):
    x = SeededOperand(11, 37, 29, transposed)
    full = x.full()
    assert full.shape == x.shape
    idx = [0, 5, x.shape[0] - 1]
    np.testing.assert_array_equal(x.rows(idx), full[idx, :])
    jdx = [1, x.shape[1] - 1, 3]
    np.testing.assert_array_equal(x.cols(jdx), full[:, jdx])
    # Same numbers as the contiguous generator in storage order.
    flat = oracle.fill_uniform(37 * 29, 11)
    stored = flat.reshape(29, 37).T
    np.testing.assert_array_equal(full, stored.T if transposed else stored)


def test_positions_cover_every_tile():
    rows, cols, ri, rj = spread_positions(1000, 700, 128, 96, seed=3, randoms=50)
    assert sorted({i // 128 for i in rows}) == list(range(8))
    assert sorted({j // 96 for j in cols}) == list(range(8))
    assert all(0 <= i < 1000 for i in rows) and all(0 <= j < 700 for j in cols)
    assert len(ri) == len(rj) == 50


M, N, K, TM, TN = 300, 260, 70, 64, 48


@pytest.fixture(scope="module")
def product():
    a = SeededOperand(21, M, K, False)
    b = SeededOperand(22, N, K, True)  # op T: stored N x K
    c = (a.full().astype(np.float64) @ b.full().astype(np.float64)).astype(np.float32)
    return a, b, np.asfortranarray(c)


def reader(c):
    return lambda j0, j1: c[:, j0:j1]


def test_correct_product_passes(product):
    a, b, c = product
    res = spread_check(a, b, reader(c), TM, TN, seed=1, randoms=200, slab_bytes=M * 4 * 37)
    assert res["violations"] == 0
    assert res["elements"] == M * 6 + N * 5 + 200
    assert res["tile_grid"] == [5, 6]


def planted(c, kind):
    bad = c.copy()
    if kind == "swapped_blocks":   # C tiles (1,2) and (3,4) exchanged
        t1 = bad[TM:2 * TM, 2 * TN:3 * TN].copy()
        bad[TM:2 * TM, 2 * TN:3 * TN] = bad[3 * TM:4 * TM, 4 * TN:5 * TN]
        bad[3 * TM:4 * TM, 4 * TN:5 * TN] = t1
    elif kind == "stale_block":    # one tile never written (zeros)
        bad[2 * TM:3 * TM, TN:2 * TN] = 0
    elif kind == "shifted_block":  # one tile written one column off
        bad[0:TM, 3 * TN + 1:4 * TN] = c[0:TM, 3 * TN:4 * TN - 1]
    elif kind == "half_k":         # one tile missing its last K panel
        bad[4 * TM:M, 5 * TN:N] *= 0.5
    return bad


@pytest.mark.parametrize("kind", ["swapped_blocks", "stale_block", "shifted_block", "half_k"])
def test_planted_block_mistakes_fail(product, kind):
    a, b, c = product
    res = spread_check(a, b, reader(planted(c, kind)), TM, TN, seed=1, randoms=200)
    assert res["violations"] > 0, kind
