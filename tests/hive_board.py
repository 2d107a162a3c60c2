"""Hand-built Hive positions in the reference's 3424-byte state layout.

Test helper only.  Cells use the reference's fixed 23x23 grid centred on
axial (0, 0): cell = (r + 11) * 23 + (q + 11) (hive_gpu/csrc/hex_grid.cuh:8-15).
"""
from __future__ import annotations

import numpy as np

GRID, HALF = 23, 11
OFF_HEIGHT, OFF_OCC, OFF_WTOP, OFF_BTOP = 2645, 3176, 3248, 3320
OFF_QUEEN, OFF_HANDS, OFF_TURN, OFF_QPLACED, OFF_RESULT, OFF_STUN = 3392, 3396, 3412, 3414, 3415, 3416
Q, A, G, S, B, M, L, P = range(1, 9)
WHITE, BLACK = 0, 1
PER_TYPE = [1, 3, 3, 2, 2, 1, 1, 1]
DIRS = [(1, 0), (1, -1), (0, -1), (-1, 0), (-1, 1), (0, 1)]  # E NE NW W SW SE as (dq, dr)


def cell(q: int, r: int) -> int:
    return (r + HALF) * GRID + (q + HALF)


def qr(c: int):
    return c % GRID - HALF, c // GRID - HALF


def _u16(s, off, v):
    s[off] = v & 0xFF
    s[off + 1] = (v >> 8) & 0xFF


def _bit(s, base, c, on):
    byte = base + (c >> 3)
    if on:
        s[byte] |= 1 << (c & 7)
    else:
        s[byte] &= ~(1 << (c & 7)) & 0xFF


def empty_state(mask: int = 0, turn: int = 0) -> np.ndarray:
    s = np.zeros(3424, np.uint8)
    _u16(s, OFF_QUEEN, 0xFFFF)
    _u16(s, OFF_QUEEN + 2, 0xFFFF)
    for c in (WHITE, BLACK):
        for t in range(5):
            s[OFF_HANDS + c * 8 + t] = PER_TYPE[t]
        s[OFF_HANDS + c * 8 + 5] = 1 if mask & 1 else 0
        s[OFF_HANDS + c * 8 + 6] = 1 if mask & 2 else 0
        s[OFF_HANDS + c * 8 + 7] = 1 if mask & 4 else 0
    _u16(s, OFF_STUN, 0xFFFF)
    _u16(s, OFF_TURN, turn)
    return s


def put(s: np.ndarray, q: int, r: int, pt: int, colour: int, from_hand: bool = True) -> None:
    """Push a piece onto the stack at (q, r), keeping every derived field consistent."""
    c = cell(q, r)
    h = int(s[OFF_HEIGHT + c])
    s[h * 529 + c] = pt | (colour << 4)
    s[OFF_HEIGHT + c] = h + 1
    _bit(s, OFF_OCC, c, True)
    _bit(s, OFF_WTOP, c, colour == WHITE)
    _bit(s, OFF_BTOP, c, colour == BLACK)
    if pt == Q:
        _u16(s, OFF_QUEEN + 2 * colour, c)
        s[OFF_QPLACED] |= 1 << colour
    if from_hand:
        s[OFF_HANDS + colour * 8 + pt - 1] -= 1


def set_turn(s: np.ndarray, turn: int) -> None:
    _u16(s, OFF_TURN, turn)


def set_stun(s: np.ndarray, c: int) -> None:
    _u16(s, OFF_STUN, c)


def moves_as_set(moves: np.ndarray, n: int):
    """{(type, piece, from, to)} of the first n 6-byte moves."""
    m = moves[:n].astype(np.int64)
    return {(int(x[0]), int(x[1]), int(x[2] | (x[3] << 8)), int(x[4] | (x[5] << 8))) for x in m}


def dests_of(moves: np.ndarray, n: int, from_cell: int):
    return {t for (ty, _, f, t) in moves_as_set(moves, n) if ty == 1 and f == from_cell}
