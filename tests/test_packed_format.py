"""The packed low-bit format's NumPy statement (tests/packed_ref.py) on the
CPU: exact round trip on structured weights (+-0, one-valued and empty
groups, a ragged last block), its status bits, and the bits-per-weight
figure."""
import numpy as np

from packed_ref import pack_ref, structured, unpack_ref


def test_round_trip_exact():
    q, masks = structured(37, 300, seed=1)
    codes, lut, sal, st = pack_ref(q.view(np.uint16), masks)
    assert st == 0
    assert np.array_equal(unpack_ref(codes, lut, sal, 300), q.view(np.uint16))
    # the +-0 pairs survive as distinct values
    assert (q.view(np.uint16) == 0x8000).any() and (q.view(np.uint16) == 0).any()


def test_lut_layout_ascending_per_group():
    q, masks = structured(5, 128, seed=2)
    codes, lut, sal, st = pack_ref(q.view(np.uint16), masks)
    vals = lut.view(np.float16).astype(np.float64)
    for r in range(5):
        for lo, hi in ((0, 2), (2, 4), (4, 8)):
            assert np.all(np.diff(vals[r, 0, lo:hi]) >= 0)


def test_status_bits():
    q, masks = structured(8, 256, seed=3)
    bad = q.copy()
    row, col = 2, int(np.nonzero(masks[2, :128] == 1)[0][0])
    bad[row, col] = np.float16(0.123)          # a third value in a 2-value group
    assert pack_ref(bad.view(np.uint16), masks)[3] & 1
    m2 = masks.copy()
    c = int(np.nonzero(masks[0, :128] == 3)[0][0])
    m2[5, c] = 1                               # salient column not shared by row 5
    assert pack_ref(q.view(np.uint16), m2)[3] & 2
    m3 = masks.copy()
    m3[1, 7] = 0
    assert pack_ref(q.view(np.uint16), m3)[3] & 4


def test_bits_per_weight():
    R, C = 4096, 16384
    nblk = C // 128
    bits = (R * nblk * 32 + R * nblk * 8 * 2 + nblk * 16) * 8 / (R * C)
    assert abs(bits - 3.0) < 0.01
