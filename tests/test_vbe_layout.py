"""CPU checks of the VBE test layout (tests/tbe_helpers.VbeCase) against a
small case worked out by hand, so the GPU VBE tests rest on a checked
construction."""

import numpy as np

from tbe_helpers import VbeCase


def test_vbe_layout_hand_case():
    # T=2 features, R=3 ranks; D = 8, 4.
    c = VbeCase(np.random.default_rng(0), [[3, 0, 2], [1, 4, 1]], [8, 4], [10, 20], 5)
    assert c.total_B == 11 and c.max_B == 6
    assert c.B_offsets.tolist() == [0, 5, 11]
    assert c.rpf.tolist() == [[0, 3, 3, 5], [0, 1, 5, 6]]
    # (rank, feature) blocks: r0: 3x8, 1x4; r1: 0x8, 4x4; r2: 2x8, 1x4
    assert c.out_ofr.tolist() == [0, 24, 28, 28, 44, 60, 64]
    assert c.row_out.tolist() == [0, 8, 16, 44, 52, 24, 28, 32, 36, 40, 60]
    assert c.bag_b.tolist() == [0, 1, 2, 3, 4, 0, 1, 2, 3, 4, 5]
    assert c.b_t_map(26).tolist()[5] == (1 << 26) | 0
    # dense padding: table 0 has 5 real bags of 6, table 1 all 6
    lens = np.diff(c.dense.offsets)
    assert lens[5] == 0 and lens[:5].tolist() == np.diff(c.offsets)[:5].tolist()
    d = np.arange(6 * 12, dtype=np.float32).reshape(6, 12)
    flat = c.dense_to_flat(d)
    assert flat[44:52].tolist() == d[3, 0:8].tolist()   # table 0, b=3 (rank 2, b_r 0)
    assert flat[60:64].tolist() == d[5, 8:12].tolist()  # table 1, b=5 (rank 2)
    assert np.array_equal(c.dense_to_flat(c.flat_to_dense(flat)), flat)
