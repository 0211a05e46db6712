"""The packed low-bit format's NumPy statement (tests/packed_ref.py) on the
CPU: exact round trip on structured weights (+-0, one-valued and empty
groups, a ragged last block, out-of-table values kept as exceptions), the
table choice, its status bits, and the bits-per-weight figure."""
import numpy as np

from packed_ref import pack_ref, structured, unpack_ref


def test_round_trip_exact():
    q, masks = structured(37, 300, seed=1)
    codes, lut, sal, ex, st = pack_ref(q.view(np.uint16), masks)
    assert st == 0 and len(ex[0]) == 0
    assert np.array_equal(unpack_ref(codes, lut, sal, 300), q.view(np.uint16))
    # the +-0 pairs survive as distinct values
    assert (q.view(np.uint16) == 0x8000).any() and (q.view(np.uint16) == 0).any()


def test_round_trip_with_exceptions():
    q, masks = structured(37, 300, seed=4, n_odd=9)
    bits = q.view(np.uint16)
    codes, lut, sal, ex, st = pack_ref(bits, masks)
    assert st == 0 and 1 <= len(ex[0]) <= 9
    assert np.array_equal(unpack_ref(codes, lut, sal, 300, ex), bits)
    # without the exceptions exactly those elements differ
    diff = np.nonzero((unpack_ref(codes, lut, sal, 300) != bits).ravel())[0]
    assert np.array_equal(diff, ex[0])
    # delta = value - the entry the element's code decodes to, in fp32
    plain = unpack_ref(codes, lut, sal, 300).ravel()
    want = bits.ravel()[ex[0]].view(np.float16).astype(np.float32) - \
        plain[ex[0]].view(np.float16).astype(np.float32)
    assert np.array_equal(ex[2], want)


def test_table_keeps_most_frequent():
    """A group with values a (x3), b (x2), c (x1) keeps a and b (ascending)
    and makes c the exception, whatever the key order."""
    R, C = 1, 128
    masks = np.ones((R, C), np.uint8)
    q = np.zeros((R, C), np.float16)
    masks[0, 6:] = 2                           # group 1 = columns 0..5
    q[0, :6] = np.array([0.5, -0.25, 0.5, 0.75, 0.5, 0.75], np.float16)   # c = -0.25 once
    q[0, 6:] = np.float16(0.1)
    codes, lut, sal, ex, st = pack_ref(q.view(np.uint16), masks)
    assert st == 0
    assert list(lut[0, 0, :2].view(np.float16)) == [0.5, 0.75]
    assert list(ex[0]) == [1]
    assert ex[2][0] == np.float32(-0.25) - np.float32(0.5)


def test_lut_layout_ascending_per_group():
    q, masks = structured(5, 128, seed=2)
    codes, lut, sal, ex, st = pack_ref(q.view(np.uint16), masks)
    vals = lut.view(np.float16).astype(np.float64)
    for r in range(5):
        for lo, hi in ((0, 2), (2, 4), (4, 8)):
            assert np.all(np.diff(vals[r, 0, lo:hi]) >= 0)


def test_status_bits():
    q, masks = structured(8, 256, seed=3)
    bad = q.copy()
    row, col = 2, int(np.nonzero(masks[2, :128] == 1)[0][0])
    bad[row, col] = np.float16(0.123)          # a third value in a 2-value group: an exception
    codes, lut, sal, ex, st = pack_ref(bad.view(np.uint16), masks)
    assert st == 0 and list(ex[0]) == [row * 256 + col]
    assert pack_ref(bad.view(np.uint16), masks, ex_cap=0)[4] & 1     # list overflow
    m2 = masks.copy()
    c = int(np.nonzero(masks[0, :128] == 3)[0][0])
    m2[5, c] = 1                               # salient column not shared by row 5
    assert pack_ref(q.view(np.uint16), m2)[4] & 2
    m3 = masks.copy()
    m3[1, 7] = 0
    assert pack_ref(q.view(np.uint16), m3)[4] & 4


def test_bits_per_weight():
    R, C = 4096, 16384
    nblk = C // 128
    bits = (R * nblk * 32 + R * nblk * 8 * 2 + nblk * 16) * 8 / (R * C)
    assert abs(bits - 3.0) < 0.01
