"""The packed block-record layout restated in oracle/pool_format.py agrees with the
layout documented in include/heterokv.h (hand-placed nibbles) and round-trips.  CPU only."""
import numpy as np

from oracle import pool_format as pf


def test_nibble_positions():
    assert [pf.nib_shift(k) for k in range(8)] == [0, 16, 4, 20, 8, 24, 12, 28]


def test_k_row_word_layout_by_hand():
    codes = np.zeros(128, dtype=np.uint8)
    codes[8:16] = [1, 2, 3, 4, 5, 6, 7, 8]  # word 1 = dims 8..15
    packed = pf.pack_k_rows(codes)
    w = packed.view("<u4")
    assert w[0] == 0
    # x0..x7 = 1..8 at bits 0,16,4,20,8,24,12,28
    expect = (1 << 0) | (2 << 16) | (3 << 4) | (4 << 20) | (5 << 8) | (6 << 24) | (7 << 12) | (8 << 28)
    assert int(w[1]) == expect
    # the unpack trick: (w >> 4i) & 0x000F000F gives the natural pairs (d2i, d2i+1)
    for i in range(4):
        pair = (int(w[1]) >> (4 * i)) & 0x000F000F
        assert (pair & 0xF, pair >> 16) == (codes[8 + 2 * i], codes[8 + 2 * i + 1])


def test_v_word_layout_by_hand():
    codes = np.zeros((16, 128), dtype=np.uint8)
    # tokens 4..7 (g=1) at dim c=3 + 32*m (m=2 -> dim 67) and dim 83 (= 67 + 16)
    codes[4:8, 67] = [1, 2, 3, 4]
    codes[4:8, 83] = [5, 6, 7, 8]
    w = pf.pack_v_block(codes).view("<u4")
    idx = (1 * 16 + 3) * 4 + 2
    expect = (1 << 0) | (2 << 16) | (3 << 4) | (4 << 20) | (5 << 8) | (6 << 24) | (7 << 12) | (8 << 28)
    assert int(w[idx]) == expect
    assert np.count_nonzero(w) == 1


def test_round_trips_random():
    rng = np.random.default_rng(0)
    k = rng.integers(0, 16, (16, 128), dtype=np.uint8)
    assert np.array_equal(pf.unpack_k_rows(pf.pack_k_rows(k)), k)
    assert np.array_equal(pf.unpack_v_block(pf.pack_v_block(k)), k)


def test_record_offsets_and_size():
    assert pf.record_bytes(8) == 17664 and pf.record_bytes(4) == 8832
    o = pf.offsets(8)
    assert (o["vc"], o["ks"], o["vs"], o["kz"], o["vz"]) == (8192, 16384, 16896, 17408, 17536)


def test_v_tile_layout():
    v = np.arange(16 * 128, dtype=np.float32).reshape(16, 128)
    t = pf.v_tile(v)
    # [g][c][n][i] = V[4g+i][c+16n]
    assert t[2, 5, 3, 1] == v[9, 53]
