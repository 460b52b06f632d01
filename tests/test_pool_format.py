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
    # head i's part starts at i * 2208; inside it K codes, V codes, K scales, V scales,
    # K zps, V zps (1024 + 1024 + 64 + 64 + 16 + 16 bytes)
    o = pf.offsets(0)
    assert (o["kc"], o["vc"], o["ks"], o["vs"], o["kz"], o["vz"]) == (0, 1024, 2048, 2112, 2176, 2192)
    o = pf.offsets(5)
    assert (o["kc"], o["vz"]) == (11040, 11040 + 2192)
    assert o["vz"] + 16 == pf.offsets(6)["kc"]


def test_record_parts_are_contiguous_per_head():
    rng = np.random.default_rng(3)
    H = 3
    kc = rng.integers(0, 16, (H, 16, 128), dtype=np.uint8)
    vc = rng.integers(0, 16, (H, 16, 128), dtype=np.uint8)
    ks, vs = rng.random((H, 16), dtype=np.float32), rng.random((H, 16), dtype=np.float32)
    kz, vz = rng.integers(0, 16, (H, 16), dtype=np.uint8), rng.integers(0, 16, (H, 16), dtype=np.uint8)
    rec = pf.build_record(kc, vc, ks, vs, kz, vz)
    for i in range(H):
        one = pf.build_record(kc[i:i + 1], vc[i:i + 1], ks[i:i + 1], vs[i:i + 1], kz[i:i + 1], vz[i:i + 1])
        assert np.array_equal(rec[i * 2208:(i + 1) * 2208], one)


def test_v_tile_layout():
    v = np.arange(16 * 128, dtype=np.float32).reshape(16, 128)
    t = pf.v_tile(v)
    # [g][c][n][i] = V[4g+i][c+16n]
    assert t[2, 5, 3, 1] == v[9, 53]
