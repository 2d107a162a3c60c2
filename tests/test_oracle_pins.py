"""Pins of the CPU oracle that do not come from the reference's golden vectors.

Each test checks the oracle against something the mathematics or the
reference's own test suite fixes, chosen so a plausible slip (wrong
direction order, flipped sign, off-by-one in rounding, transposed
coordinates) fails:

* hex neighbour table      -- closed form of hive_gpu/csrc/hex_grid.cuh:41-49,69-108
* articulation points      -- brute force (delete vertex, flood fill) incl. disconnected hives,
                              semantics of articulation.cuh:34-168 (DFS from the lowest cell only)
* centroid rounding        -- Python's round() (banker's), state_encoder.cuh:55-79,889-906
* action index             -- independent restatement of mcts_tree.cuh:146-179 and the
                              reference's own Python fallback hive_gpu/__init__.py:109-141
* Philox4x32-10            -- Random123 known-answer vectors
* rule cases               -- tests/test_gpu_move_gen.py:148-160 and the board rules of
                              tests/test_board.py / test_expansion_pieces.py, compared as sets
"""
import random
from fractions import Fraction

import numpy as np
import pytest

import hive_board as hb


def test_neighbor_table_closed_form(oracle):
    nb = oracle.neighbor_table()
    for c in range(529):
        q, r = hb.qr(c)
        for d, (dq, dr) in enumerate(hb.DIRS):
            q2, r2 = q + dq, r + dr
            inside = -11 <= q2 <= 11 and -11 <= r2 <= 11
            assert nb[c, d] == (hb.cell(q2, r2) if inside else -1)


def _random_hive(rng, n, connected=True):
    cells = [(0, 0)]
    while len(cells) < n:
        if connected:
            q, r = rng.choice(cells)
            dq, dr = rng.choice(hb.DIRS)
            c = (q + dq, r + dr)
        else:
            c = (rng.randint(-6, 6), rng.randint(-6, 6))
        if c not in cells:
            cells.append(c)
    return cells


def _brute_ap(cells):
    """Articulation points of the component containing the lowest cell index."""
    idx = {hb.cell(q, r) for q, r in cells}
    if len(idx) <= 2:
        return set()

    def nbrs(c):
        q, r = hb.qr(c)
        return [hb.cell(q + dq, r + dr) for dq, dr in hb.DIRS
                if -11 <= q + dq <= 11 and -11 <= r + dr <= 11 and hb.cell(q + dq, r + dr) in idx]

    def flood(start, banned):
        seen, todo = {start}, [start]
        while todo:
            x = todo.pop()
            for y in nbrs(x):
                if y != banned and y not in seen:
                    seen.add(y)
                    todo.append(y)
        return seen

    comp = flood(min(idx), None)
    out = set()
    for v in comp:
        rest = comp - {v}
        if not rest:
            continue
        if flood(min(rest), v) != rest:
            out.add(v)
    return out


@pytest.mark.parametrize("connected", [True, False])
def test_articulation_brute_force(oracle, connected):
    rng = random.Random(7 if connected else 8)
    for trial in range(300):
        cells = _random_hive(rng, rng.randint(1, 28), connected)
        s = hb.empty_state()
        for q, r in cells:
            hb.put(s, q, r, hb.A, trial & 1, from_hand=False)
        words = oracle.articulation(s)
        got = {w * 64 + b for w in range(9) for b in range(64) if (int(words[w]) >> b) & 1}
        assert got == _brute_ap(cells), (trial, cells)


def _py_round_centroid(cells):
    if not cells:
        return 0, 0
    return (round(Fraction(sum(q for q, _ in cells), len(cells))),
            round(Fraction(sum(r for _, r in cells), len(cells))))


def test_centroid_bankers_rounding(oracle):
    rng = random.Random(3)
    for _ in range(400):
        cells = list({(rng.randint(-11, 11), rng.randint(-11, 11)) for _ in range(rng.randint(0, 6))})
        s = hb.empty_state()
        for q, r in cells:
            hb.put(s, q, r, hb.B, 0, from_hand=False)
        assert oracle.centroid(s) == _py_round_centroid(cells)
    # exact .5 ties in both directions: 0.5 -> 0, 1.5 -> 2, -0.5 -> 0, -1.5 -> -2
    for cells, want in [([(0, 0), (1, 0)], 0), ([(1, 0), (2, 0)], 2), ([(0, 0), (-1, 0)], 0),
                        ([(-1, 0), (-2, 0)], -2)]:
        s = hb.empty_state()
        for q, r in cells:
            hb.put(s, q, r, hb.B, 0, from_hand=False)
        assert oracle.centroid(s)[0] == want


def _action(mtype, pt, frm, to, cq, cr):
    """Independent statement of the 85,834-wide action index (ENC_GRID = 17)."""
    if mtype == 2:
        return 85833

    def win(c):
        q, r = hb.qr(c)
        col, row = q - cq + 8, r - cr + 8
        return row * 17 + col if 0 <= col < 17 and 0 <= row < 17 else None

    if mtype == 0:
        w = win(to)
        return -1 if w is None else (pt - 1) * 289 + w
    a, b = win(frm), win(to)
    return -1 if a is None or b is None else 2312 + a * 289 + b


def test_action_index_formula(oracle):
    rng = random.Random(11)
    for _ in range(3000):
        mtype = rng.choice([0, 1, 2])
        pt, frm, to = rng.randint(1, 8), rng.randint(0, 528), rng.randint(0, 528)
        cq, cr = rng.randint(-11, 11), rng.randint(-11, 11)
        mv = np.array([mtype, pt, frm & 255, frm >> 8, to & 255, to >> 8], np.uint8)
        assert oracle.move_to_action(mv, cq, cr) == _action(mtype, pt, frm, to, cq, cr)


def test_philox_known_answers(oracle):
    kat = [((0, 0), (0, 0, 0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
           ((0xFFFFFFFF, 0xFFFFFFFF), (0xFFFFFFFF,) * 4, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
           ((0xA4093822, 0x299F31D0), (0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344),
            (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1))]
    for key, ctr, want in kat:
        assert tuple(int(x) for x in oracle.philox(key[0], key[1], ctr)) == want


# ---- rule cases -------------------------------------------------------------

def test_initial_position(oracle):
    """tests/test_gpu_move_gen.py:148-160: 4 placements at turn 0, result 0."""
    s = oracle.init_state(0)
    moves, n = oracle.legal_moves(s)
    assert n == 4
    assert hb.moves_as_set(moves, n) == {(0, t, 0, hb.cell(0, 0)) for t in (2, 3, 4, 5)}
    assert s[hb.OFF_RESULT] == 0
    s7 = oracle.init_state(7)
    assert oracle.legal_moves(s7)[1] == 7  # A G S B M L P, no queen on the first turn


def _white_to_move_after_queens():
    """White Q at (0,0), black Q at (1,0); white to move at turn 4 (own queen placed)."""
    s = hb.empty_state()
    hb.put(s, 0, 0, hb.Q, hb.WHITE)
    hb.put(s, 1, 0, hb.Q, hb.BLACK)
    hb.set_turn(s, 4)
    return s


def test_grasshopper_jumps_line(oracle):
    s = _white_to_move_after_queens()
    hb.put(s, -1, 0, hb.G, hb.WHITE)
    hb.put(s, 2, 0, hb.A, hb.BLACK)
    moves, n = oracle.legal_moves(s)
    assert hb.dests_of(moves, n, hb.cell(-1, 0)) == {hb.cell(3, 0)}  # jumps Q, Q, A in a line


def test_spider_exactly_three(oracle):
    s = _white_to_move_after_queens()
    hb.put(s, -1, 0, hb.S, hb.WHITE)
    moves, n = oracle.legal_moves(s)
    d = hb.dests_of(moves, n, hb.cell(-1, 0))
    # around the 2-cell line Q(0,0) Q(1,0) the spider walks three cells either way
    assert d == {hb.cell(2, -1), hb.cell(1, 1)}


def test_pinned_middle_piece(oracle):
    s = _white_to_move_after_queens()
    hb.put(s, -1, 0, hb.A, hb.WHITE)
    hb.put(s, -2, 0, hb.A, hb.WHITE)
    moves, n = oracle.legal_moves(s)
    assert hb.dests_of(moves, n, hb.cell(-1, 0)) == set()  # articulation point, height 1
    assert hb.dests_of(moves, n, hb.cell(0, 0)) == set()


def test_beetle_climbs_and_queen_must_be_placed(oracle):
    s = _white_to_move_after_queens()
    hb.put(s, -1, 0, hb.B, hb.WHITE)
    moves, n = oracle.legal_moves(s)
    assert hb.cell(0, 0) in hb.dests_of(moves, n, hb.cell(-1, 0))  # climbs onto own queen
    t = hb.empty_state()
    hb.put(t, 0, 0, hb.A, hb.WHITE)
    hb.put(t, 1, 0, hb.A, hb.BLACK)
    hb.put(t, -1, 0, hb.G, hb.WHITE)
    hb.put(t, 2, 0, hb.G, hb.BLACK)
    hb.put(t, -2, 0, hb.S, hb.WHITE)
    hb.put(t, 3, 0, hb.S, hb.BLACK)
    hb.set_turn(t, 6)  # white's 4th turn without a queen: queen placements only
    moves, n = oracle.legal_moves(t)
    assert {m[1] for m in hb.moves_as_set(moves, n)} == {hb.Q}


def test_pillbug_throws_enemy_and_mosquito_copies(oracle):
    s = hb.empty_state(mask=7)
    hb.put(s, 0, 0, hb.Q, hb.WHITE)
    hb.put(s, 1, 0, hb.P, hb.WHITE)
    hb.put(s, 2, 0, hb.A, hb.BLACK)
    hb.put(s, 3, 0, hb.Q, hb.BLACK)
    hb.set_turn(s, 4)
    moves, n = oracle.legal_moves(s)
    ms = hb.moves_as_set(moves, n)
    # throwing the black ant at (2,0) would split the hive: pinned, no throw;
    # the white queen at (0,0) is a leaf: the pillbug may throw it
    assert not any(f == hb.cell(2, 0) for (_, _, f, _) in ms)
    throws_q = {t for (ty, pt, f, t) in ms if f == hb.cell(0, 0) and pt == hb.Q}
    # (2,-1) and (1,1) are two steps from the queen: only a throw reaches them
    assert {hb.cell(2, -1), hb.cell(1, 1)} <= throws_q
    # a ground mosquito next to an ant copies ant moves
    m = hb.empty_state(mask=7)
    hb.put(m, 0, 0, hb.Q, hb.WHITE)
    hb.put(m, 1, 0, hb.Q, hb.BLACK)
    hb.put(m, -1, 0, hb.M, hb.WHITE)
    hb.put(m, 2, 0, hb.A, hb.BLACK)
    hb.set_turn(m, 4)
    moves, n = oracle.legal_moves(m)
    # next to the white queen only: the mosquito slides one step like a queen
    assert hb.dests_of(moves, n, hb.cell(-1, 0)) == {hb.cell(0, -1), hb.cell(-1, 1)}
    hb.put(m, -1, 1, hb.A, hb.BLACK)  # now also next to an ant: ant reach joins the union
    hb.set_turn(m, 4)
    moves, n = oracle.legal_moves(m)
    assert len(hb.dests_of(moves, n, hb.cell(-1, 0))) > 2


def test_site_perimeter_bound():
    """A connected n-cell hive has at most 2n + 4 empty neighbour cells.

    The engine sizes its per-piece destination buffers with this bound (an
    ant's destinations are such cells of the hive without the ant)."""
    rng = random.Random(7)
    worst = {}
    for _ in range(3000):
        n = rng.randint(1, 27)
        cells = set(_random_hive(rng, n))
        per = {(q + dq, r + dr) for q, r in cells for dq, dr in hb.DIRS} - cells
        assert len(per) <= 2 * n + 4
        worst[n] = max(worst.get(n, 0), len(per))
    # a straight line reaches the bound
    line = {(i, 0) for i in range(10)}
    assert len({(q + dq, r + dr) for q, r in line for dq, dr in hb.DIRS} - line) == 24


def test_destination_counts_within_buffers(oracle):
    """Legal lists of seeded random-play positions: per-piece destination
    counts stay inside the engine's buffers (ant < 64, mosquito <= 128,
    spider / ladybug <= 32).  A piece's own moves are one contiguous run of
    MOVE entries with its cell as source (throws come after all pieces)."""
    worst = {}
    for mask, max_ply in ((0, 120), (7, 150)):
        st, _ = oracle.generate_positions(4096, mask, max_ply, 0xB0B)
        moves, n, _, _ = oracle.batch_legal_features_actions(st, want_features=False, want_actions=False)
        for i in range(st.shape[0]):
            m = moves[i, :n[i]]
            key = [(int(r[1]), int(r[2]) | (int(r[3]) << 8)) if r[0] == 1 else None for r in m]
            run, seen = 0, set()
            for j, k in enumerate(key):
                run = run + 1 if j > 0 and k is not None and k == key[j - 1] else 1
                if k is not None and (j + 1 == len(key) or key[j + 1] != k) and k not in seen:
                    seen.add(k)
                    worst[k[0]] = max(worst.get(k[0], 0), run)
    assert worst.get(2, 0) < 64 and worst.get(6, 0) <= 128
    assert worst.get(4, 0) <= 32 and worst.get(7, 0) <= 32
    assert worst.get(2, 0) > 20  # the sample does exercise long ant searches
