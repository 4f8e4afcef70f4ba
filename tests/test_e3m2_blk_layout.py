"""Host helpers of the block-packed E3M2 layout (FMT_E3M2_BLK): the 6-bit field of each row
of a 32-row block, and the numpy packing the GPU tests use to pack the oracle's codes."""
import numpy as np

import mxfa

# Row held by each 6-bit field of a block (fields 0..15: rows with bit 2 clear, 16..31: set)
ROW_OF_FIELD = [0, 1, 2, 3, 8, 9, 10, 11, 16, 17, 18, 19, 24, 25, 26, 27,
                4, 5, 6, 7, 12, 13, 14, 15, 20, 21, 22, 23, 28, 29, 30, 31]


def test_pack_helpers_match_the_bit_layout():
    """e3m2_to_blk against the layout read off one
    192-bit integer per block, and its inverse."""
    assert [mxfa.blk_field(r) for r in ROW_OF_FIELD] == list(range(32))
    rng = np.random.default_rng(600)
    c = rng.integers(0, 64, (2, 96, 12), dtype=np.uint8)
    b = mxfa.e3m2_to_blk(c)
    assert b.shape == (2, 3, 12, 24)
    for m, nb, col in [(0, 0, 0), (1, 2, 11), (0, 1, 5)]:
        big = int.from_bytes(bytes(b[m, nb, col]), "little")
        assert [(big >> (6 * f)) & 63 for f in range(32)] == [c[m, 32 * nb + r, col] for r in ROW_OF_FIELD]
    np.testing.assert_array_equal(mxfa.e3m2_from_blk(b), c)
