"""The engine's device programs run on the CPU under the wave emulator.

tests/emu/ compiles hive_neuralnet_amd/csrc/hive_phases.hpp for the host,
running each 64-lane wave as 64 threads with barrier-based shuffles and
ballots.  This checks the device logic (order of emission, features,
compact successor summaries, queen escape) against the reference's golden
vectors without a GPU; the GPU tests check the compiled HIP library itself.
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT, load_golden

EMU = os.path.join(ROOT, "tests", "emu")


@pytest.fixture(scope="module")
def emu():
    import fcntl
    # one build at a time when test processes run side by side (the library is
    # renamed into place, so a loader never sees a partly written file)
    with open(os.path.join(EMU, ".build.lock"), "w") as lock:
        fcntl.flock(lock, fcntl.LOCK_EX)
        subprocess.run(["make", "-s", "-C", EMU], check=True)
        fcntl.flock(lock, fcntl.LOCK_UN)
    return ctypes.CDLL(os.path.join(EMU, "libwave_emu.so"))


@pytest.fixture(scope="module")
def emu_antgrp(emu):
    """The emulator build whose lane groups finish the ant searches (HW_ANT_GROUP=1)."""
    return ctypes.CDLL(os.path.join(EMU, "libwave_emu_antgrp.so"))


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


@pytest.mark.parametrize("name", ["c1", "c2", "c3"])
def test_emulated_legal_features(emu, oracle, name):
    g = load_golden(name)
    st = np.ascontiguousarray(g["states"][:47])
    B = len(st)
    mv = np.zeros((B, 256, 6), np.uint8)
    n = np.zeros(B, np.int32)
    f = np.zeros((B, 122), np.float32)
    a = np.zeros((B, 256), np.int32)
    emu.emu_legal(_p(st), ctypes.c_int64(B), _p(mv), _p(n), _p(f), _p(a))
    assert np.array_equal(n, g["n"][:B])
    assert np.array_equal(mv, g["moves"][:B])
    assert np.array_equal(f.view(np.uint32), g["features"][:B].view(np.uint32))
    _, _, _, oa = oracle.batch_legal_features_actions(st)
    assert np.array_equal(a, oa)


@pytest.mark.parametrize("mask,start_ply,seed", [(0, 0, 81), (0, 40, 82), (7, 60, 83)])
def test_emulated_board_resident_play(emu, oracle, mask, start_ply, seed):
    """k_random_play's ply loop: the board stays in LDS, each ply's move is
    decoded from the generated tables (list_slot) rather than read from an
    emitted list, and the state row only receives the bytes that changed
    (apply_mirrored).  After 40 plies of given choices the rows and the ply
    counts equal the oracle's replay: its own legal list, slot
    (u * n) >> 32, apply_move, stopping at a result."""
    B, plies = 24, 40
    states, _ = oracle.generate_positions(B, mask, start_ply, seed, threads=4)
    states = np.ascontiguousarray(states)
    u = np.random.default_rng(seed).integers(0, 2**32, size=(B, plies), dtype=np.uint64).astype(np.uint32)
    want = states.copy()
    want_done = np.zeros(B, np.int32)
    for i in range(B):
        s = want[i]
        for ply in range(plies):
            if s[3415] != 0:
                break
            mv, n = oracle.legal_moves(s)
            s = oracle.apply_move(s, mv[(int(u[i, ply]) * n) >> 32])
            want_done[i] += 1
        want[i] = s
    got = states.copy()
    done = np.zeros(B, np.int32)
    emu.emu_play(_p(got), ctypes.c_int64(B), ctypes.c_int(plies), _p(u), _p(done))
    assert np.array_equal(done, want_done)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("mask,max_ply,seed", [(0, 120, 71), (7, 150, 72)])
def test_emulated_group_ant_searches(emu, emu_antgrp, oracle, mask, max_ply, seed):
    """The build-time alternative whose lane group finishes each ant search
    (a batch of queued entries expanded together, one lane per entry and
    direction) against the oracle's legal lists, features and actions, on
    random-play and golden positions."""
    g = load_golden("c2" if mask == 0 else "c3")
    st, _ = oracle.generate_positions(96, mask, max_ply, seed)
    st = np.ascontiguousarray(np.concatenate([st, g["states"][:32]]))
    B = len(st)
    mv = np.zeros((B, 256, 6), np.uint8)
    n = np.zeros(B, np.int32)
    f = np.zeros((B, 122), np.float32)
    a = np.zeros((B, 256), np.int32)
    emu_antgrp.emu_legal(_p(st), ctypes.c_int64(B), _p(mv), _p(n), _p(f), _p(a))
    om, on, of, oa = oracle.batch_legal_features_actions(st)
    assert np.array_equal(n, on)
    assert np.array_equal(mv, om)
    assert np.array_equal(f.view(np.uint32), of.view(np.uint32))
    assert np.array_equal(a, oa)
    # ants: a search that ends at a target (the probes' gated lists) stops the same way
    out0 = np.zeros((B, 5), np.int32)
    out1 = np.zeros((B, 5), np.int32)
    emu.emu_gated_win(_p(st), ctypes.c_int64(B), _p(out0))
    emu_antgrp.emu_gated_win(_p(st), ctypes.c_int64(B), _p(out1))
    assert np.array_equal(out0, out1)


@pytest.mark.parametrize("name", ["c2", "c3"])
def test_emulated_successors_queen_escape(emu, name):
    g = load_golden(name)
    k = 160
    roots = np.ascontiguousarray(g["succ_root"][:k])
    idx = np.ascontiguousarray(g["succ_idx"][:k])
    st = np.ascontiguousarray(g["states"])
    mv = np.ascontiguousarray(g["moves"])
    f = np.zeros((k, 122), np.float32)
    emu.emu_successor(_p(st), _p(mv), _p(roots), _p(idx), ctypes.c_int64(k), _p(f))
    assert np.array_equal(f.view(np.uint32), g["succ_features"][:k].view(np.uint32))
    q = np.zeros(64, np.uint8)
    emu.emu_queen_escape(_p(st), ctypes.c_int64(64), _p(q))
    assert np.array_equal(q, g["queen_escape"][:64])


def test_emulated_successor_rows(emu):
    """The blocked successor program (a root's row loaded once per run of its
    rows, the board restored from registers between them) against the
    reference's successor vectors, with runs that start mid-block, a root
    that recurs after another, and out-of-range rows (zero features)."""
    g = load_golden("c2")
    k = 90
    roots = np.ascontiguousarray(g["succ_root"][:k]).copy()
    idx = np.ascontiguousarray(g["succ_idx"][:k]).copy()
    want = g["succ_features"][:k].copy()
    # a recurring root after a different one, and two bad rows
    roots = np.concatenate([roots[:7], roots[40:43], roots[7:12], [-1, roots[0]], roots[12:]])
    idx = np.concatenate([idx[:7], idx[40:43], idx[7:12], [0, 300], idx[12:]])
    want = np.concatenate([want[:7], want[40:43], want[7:12], np.zeros((2, 122), np.float32), want[12:]])
    st = np.ascontiguousarray(g["states"])
    mv = np.ascontiguousarray(g["moves"])
    n = len(roots)
    f = np.full((n, 122), np.nan, np.float32)
    roots, idx = roots.astype(np.int64), idx.astype(np.int64)
    emu.emu_successor_rows(_p(st), _p(mv), _p(roots), _p(idx), ctypes.c_int64(n), ctypes.c_int64(st.shape[0]), _p(f))
    assert np.array_equal(f.view(np.uint32), want.view(np.uint32))


def _shift_down(st, r):
    """The position moved r grid rows down (cells + 23 r): stacks, heights,
    bitboards, queen squares and the stunned cell; every piece must stay on
    the grid."""
    d = 23 * r
    out = st.copy()
    lv = st[:5 * 529].reshape(5, 529)
    out[:5 * 529] = np.concatenate([np.zeros((5, d), np.uint8), lv[:, :529 - d]], axis=1).ravel()
    h = st[2645:2645 + 529]
    assert not h[529 - d:].any()
    out[2645:2645 + 529] = np.concatenate([np.zeros(d, np.uint8), h[:529 - d]])
    for off in (3176, 3248, 3320):
        bits = np.unpackbits(st[off:off + 72], bitorder="little")[:529]
        nb = np.zeros(576, np.uint8)
        nb[d:529] = bits[:529 - d]
        out[off:off + 72] = np.packbits(nb, bitorder="little")
    for off in (3392, 3394, 3416):
        c = int(st[off]) | (int(st[off + 1]) << 8)
        if c < 529:
            c += d
            out[off], out[off + 1] = c & 255, c >> 8
    return out


def test_emulated_successor_rows_grid_edge(emu, oracle):
    """Blocked successor rows of positions moved to the bottom rows of the
    grid, where moves write cells 506-528 (cells 512-528 are the last two
    16-cell chunks, which lanes 0 and 1 restore), against the oracle's
    successor features."""
    g = load_golden("c3")
    states = []
    for st in g["states"][:40]:
        h = st[2645:2645 + 529]
        occ = np.nonzero(h)[0]
        if len(occ) < 6:
            continue
        r = 22 - int(occ.max()) // 23
        if r > 0:
            states.append(_shift_down(st, r))
        if len(states) == 3:
            break
    st = np.ascontiguousarray(np.stack(states))
    mv, n, _, _ = oracle.batch_legal_features_actions(st)
    to = mv[..., 4].astype(np.int64) | (mv[..., 5].astype(np.int64) << 8)
    assert (to >= 512).any()
    roots = np.concatenate([np.full(int(k), i, np.int64) for i, k in enumerate(n)])
    # each root's rows ordered by destination, so that moves to one cell follow
    # each other inside a run (a board not restored would keep the last one)
    idx = np.concatenate([np.argsort(to[i, :int(k)], kind="stable").astype(np.int64) for i, k in enumerate(n)])
    want = oracle.batch_successor_features(st, mv, roots, idx)
    f = np.full((len(roots), 122), np.nan, np.float32)
    mv = np.ascontiguousarray(mv)
    emu.emu_successor_rows(_p(st), _p(mv), _p(roots), _p(idx), ctypes.c_int64(len(roots)),
                           ctypes.c_int64(st.shape[0]), _p(f))
    assert np.array_equal(f.view(np.uint32), want.view(np.uint32))


def test_emulated_successor_rows_whole_lists(emu, oracle):
    """Blocked successor rows over every legal move of twelve expansion-piece
    positions in list order (runs of one root across blocks, placements that
    grow the hive by a row, moves that empty their origin, beetles that climb,
    throws), against the oracle's successor features."""
    g = load_golden("c3")
    st = np.ascontiguousarray(g["states"][40:52])
    mv, n, _, _ = oracle.batch_legal_features_actions(st)
    roots = np.concatenate([np.full(int(k), i, np.int64) for i, k in enumerate(n)])
    idx = np.concatenate([np.arange(int(k), dtype=np.int64) for k in n])
    want = oracle.batch_successor_features(st, mv, roots, idx)
    f = np.full((len(roots), 122), np.nan, np.float32)
    mv = np.ascontiguousarray(mv)
    emu.emu_successor_rows(_p(st), _p(mv), _p(roots), _p(idx), ctypes.c_int64(len(roots)),
                           ctypes.c_int64(st.shape[0]), _p(f))
    assert np.array_equal(f.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("flags,cap", [((1, 1, 1), 0), ((0, 0, 1), 0), ((1, 1, 1), 3)])
def test_emulated_root_tactical_probe(emu, flags, cap):
    """hive_probe.hpp's group programs, orchestrated as hive_probe.hip's
    launches, against the reference's probe vectors: four positions of every
    outcome kind, all stages enabled and the two-move search alone (with the
    immediate-win scan off, a root's own winning move is a two-move candidate
    whose child is a finished game with no replies: it passes).  cap 3: a
    grandchild list of three entries, so nearly every surviving candidate
    overflows it and is tested by the part programs instead (the library
    sizes the list at 256 entries per root).  The emulator runs a move
    generation in ~10 ms, so the full fixture is left to the GPU test."""
    g = load_golden("probe")
    kinds = g["kinds"]
    sel = np.concatenate([np.nonzero(kinds == k)[0][:4] for k in sorted(set(kinds.tolist()))])
    st, lm, nl, pr = (np.ascontiguousarray(g[k][sel]) for k in ("states", "legal", "nlegal", "priors"))
    B = len(st)
    j = [tuple(int(x) for x in f) for f in g["flags"]].index(flags)
    win = np.zeros(B, np.int64)
    allowed = np.zeros((B, 256), np.uint8)
    forced = np.zeros(B, np.uint8)
    emu.emu_root_probe.restype = ctypes.c_int64
    n_parts = emu.emu_root_probe(_p(st), _p(lm), _p(nl), _p(pr), ctypes.c_int64(B), *flags, _p(win), _p(allowed),
                                 _p(forced), ctypes.c_int64(cap))
    assert (n_parts > 0) == (cap > 0), n_parts  # the part programs ran exactly when the list was cut short
    assert np.array_equal(win, g["win"][j][sel]), np.nonzero(win != g["win"][j][sel])[0][:8]
    assert np.array_equal(forced, g["forced"][j][sel])
    assert np.array_equal(allowed, g["allowed"][j][sel])


def oracle_lone(oracle, s):
    """lone_empty_neighbor_of_queen (move_gen.cuh:833-851) for the opponent of
    the side to move, from the state bytes: its queen's on-grid neighbours
    hold five pieces and one empty cell, that cell; else -1."""
    del oracle
    turn = int(s[3412]) | (int(s[3413]) << 8)
    opp = (turn & 1) ^ 1
    if not (int(s[3414]) >> opp) & 1:
        return -1
    q = int(s[3392 + 2 * opp]) | (int(s[3393 + 2 * opp]) << 8)
    if q >= 529:
        return -1
    r, c = divmod(q, 23)
    nbrs = [(r + dr) * 23 + (c + dc) for dr, dc in ((0, 1), (-1, 1), (-1, 0), (0, -1), (1, -1), (1, 0))
            if 0 <= r + dr < 23 and 0 <= c + dc < 23]
    occ = [x for x in nbrs if s[2645 + x] > 0]
    empty = [x for x in nbrs if s[2645 + x] == 0]
    return empty[0] if len(occ) == 5 and len(empty) == 1 else -1


@pytest.mark.parametrize("mask,max_ply,seed", [(0, 150, 61), (7, 150, 62)])
def test_emulated_gated_immediate_win(emu, oracle, mask, max_ply, seed):
    """The probe's gated immediate-win list (WinGate) against the whole list
    on random-play positions and their children, with the target the lone
    empty neighbour of the opponent's queen (else another empty neighbour):
    ub_total bounds the whole list's length, a gated list without a winning
    move into the target means the whole list has none in its first 256
    slots, and a gated hit decides whenever ub_total <= 256."""
    st, _ = oracle.generate_positions(96, mask, max_ply, seed)
    moves, n, _, _ = oracle.batch_legal_features_actions(st)
    # children: every position's first legal moves applied, for more queens at five neighbours
    kids = []
    for i in range(len(st)):
        for k in range(min(int(n[i]), 3)):
            kids.append(oracle.apply_move(st[i], moves[i, k]))
    st = np.concatenate([st, np.stack(kids)])
    B = len(st)
    out = np.zeros((B, 5), np.int32)
    emu.emu_gated_win(_p(st), ctypes.c_int64(B), _p(out))
    cell, ub, total, hg, hf = out.T
    has = cell >= 0
    assert has.sum() > B // 2
    assert (ub[has] >= total[has]).all(), np.nonzero(has & (ub < total))[0][:8]
    assert not (hf.astype(bool) & ~hg.astype(bool)).any()  # a gated miss is a whole-list miss
    sure = hg.astype(bool) & (ub <= 256)
    assert np.array_equal(hg[sure], hf[sure])
    assert hf.sum() > 0  # the set holds immediate wins
    # the probe's own test (gated list, the whole list when the cut could matter)
    # against the whole list where the target is the queen's lone empty neighbour
    win = np.zeros(B, np.uint8)
    emu.emu_immediate_win(_p(st), ctypes.c_int64(B), _p(win))
    lone = has & (np.array([oracle_lone(oracle, s) for s in st]) == cell)
    assert np.array_equal(win[lone], hf[lone])
    assert not win[~lone].any()


@pytest.mark.parametrize("d", [3.0, 10.0, 100.0, 200.0])
def test_div_exact_matches_ieee_division(emu, d):
    """features_finish divides by 3 (hand counts), 10, 100 and 200 with
    div_exact (a reciprocal product and one residual step): every integer
    numerator below 2^24 gives the quotient IEEE division gives."""
    emu.emu_div_exact_mismatches.restype = ctypes.c_int64
    rd = np.float32(1.0) / np.float32(d)
    assert float(rd) == float(np.float32(1.0 / d))  # the literal the kernel uses
    bad = emu.emu_div_exact_mismatches(ctypes.c_int64(0), ctypes.c_int64(1 << 24),
                                       ctypes.c_float(d), ctypes.c_float(rd))
    assert bad == 0


def test_div_exact_distance_mean(emu):
    """The distance-mean feature (s / n) / 10 for piece counts n = 1..3 and
    every distance sum s below 4096, as two div_exact steps, equals the two
    IEEE divisions."""
    emu.emu_div_mean_mismatches.restype = ctypes.c_int64
    assert emu.emu_div_mean_mismatches(ctypes.c_int64(4096)) == 0


@pytest.mark.parametrize("name", ["c2", "c3"])
def test_ant_lifted_exit_lookup(emu, name):
    """The ant search reads the lifted exits of its origin's six neighbours
    from an 8-byte table by a hashed ring slot; for every occupied origin and
    every cell of the grid it equals the direct patch (exits_lifted)."""
    g = load_golden(name)
    st = np.ascontiguousarray(g["states"][:24])
    emu.emu_ring_exits_mismatches.restype = ctypes.c_int64
    assert emu.emu_ring_exits_mismatches(_p(st), ctypes.c_int64(len(st))) == 0
