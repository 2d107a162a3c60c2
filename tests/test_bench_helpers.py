"""bench.py's host helpers: the FNV-1a-64 state hash of the C4 leg."""
import numpy as np

import bench


def test_fnv1a64_known_answers():
    # published FNV-1a 64-bit test vectors
    for text, want in ((b"a", 0xAF63DC4C8601EC8C), (b"foobar", 0x85944171F73967E8)):
        row = np.frombuffer(text, np.uint8).reshape(1, -1).copy()
        assert int(bench.fnv1a64_rows(row)[0]) == want


def test_fnv1a64_masks_padding():
    rows = np.zeros((2, 3424), np.uint8)
    rows[1, 3174] = 7
    rows[1, 3421] = 9
    h = bench.fnv1a64_rows(rows)
    assert h[0] == h[1]
    rows[1, 100] = 1
    assert bench.fnv1a64_rows(rows)[1] != h[0]
