"""Known-answer cases for the Gumbel orchestrator's host logic, shared by the
numpy restatement's CPU tests and the torch orchestrator's GPU tests.

Root candidate row (fnn_mcts_orchestrator.py:339-444)
------------------------------------------------------
Hand-built positions (tests/hive_board.py), white to move (turn 8), priors
p[i] = ((7 i mod 11) + 1) / 1000 over the legal slots (ties fall to the lower
slot):

* RESERVE_B1: white queen (-2,0), grasshopper (-1,0), beetle (-1,1), ant (-3,1);
  black queen (0,0), spider (1,0), ant (1,-1).  The black queen has 4 occupied
  neighbours; only the white ant can enter its two empty neighbours (0,1) and
  (0,-1) (slots 42, 43 of 53), which makes 5, and the queen is then gated
  (both slide flanks of the last exit occupied): exactly these two qualify.
  p42 = 0.009 > p43 = 0.005 -> reserve [42, 43]; fill = the other slots by
  prior: 0.011 at slots = 3 mod 11 (3, 14, 25, 36, 47), 0.010 at slots = 6
  mod 11 (6, 17, ...) -> the row [42, 43, -1 x 4, 3, 14, 25, 36, 47, 6, 17, 28,
  39, 50].
* RESERVE_B3: white queen (2,0), ants (3,0) and (2,1), spider (3,-1); black
  queen (0,0), ant (1,0).  Eleven white moves give the black queen a second
  neighbour (slots 29 38 39 40 41 42 46 48 50 52 54).  In four of them (38, 39,
  46, 54: a white ant at (1,-1) or (0,1), touching the black ant) the queen can
  still slide away; in the other seven the white piece hangs on the queen
  alone, so the queen is an articulation point and pinned.
  - immobile only: 29 40 41 42 48 50 52 with priors .006 .006 .002 .009 .007
    .010 .002 -> the 6 reserve columns [50, 42, 48, 29, 40, 41] (52 loses the
    tie to 41 and joins the fill pool); fill [3, 14, 25, 36, 47, 6, 17, 28, 39, 9].
  - every raising move: adds 38 (.003), 39 (.010), 46 (.004), 54 (.005) ->
    reserve [39, 50, 42, 48, 29, 40]; fill [3, 14, 25, 36, 47, 6, 17, 28, 9, 20].
* CANDIDATE_SHORT (no position): 4 legal slots, priors (.1, .4, .3, .2),
  slot 2 qualifying -> reserve [2]; the fill ranks the other legal slots
  [1, 3, 0] and then every -1e30 slot in slot order: the chosen slot 2 comes
  back before the illegal 4, 5, ... -> [2, -1 x 5, 1, 3, 0, 2, 4, 5, 6, 7, 8, 9].

Sequential halving (fnn_mcts_orchestrator.py:650-731)
------------------------------------------------------
Injected candidate rows, scores base[g, s] (= Gumbel + legal logit) and the
Q each round's statistics return for a slot (formulas below, with
overrides); visits are what the rounds ran: per_slot per candidate column,
so a slot held in two columns gets twice.  The survivors of every round
(the rows passed to the next round), per_slot, the wave width and the final
choice were worked out in float64 (sigma = 50 + the batch's largest
candidate visit count); the closest kept/dropped pair of distinct slots is
0.01 apart.  The cases are built so that each of these misreadings changes
an expected value: sigma without the 50, or from the game's own visits, no
Q term, keep ceil(valid / 2), ties to the later column, per_slot from the
valid count instead of the column count, a doubled slot's visits counted
once.  Game 4 of HALVING_K16 is an exact tie (kept: the first column); game
5 needs the batch-global sigma 54 (game 1 holds slot 6 twice: 4 visits after
round 0) -- at 52 slot 30 would be kept instead of 31.
"""
from __future__ import annotations

import numpy as np

from hive_board import A, BLACK, G, Q, S, B, WHITE, empty_state, put, set_turn


def priors_formula(n):
    p = np.zeros(256, np.float32)
    i = np.arange(n)
    p[:n] = ((7 * i) % 11 + 1) / 1000.0
    return p


def reserve_b1():
    s = empty_state(0)
    put(s, -2, 0, Q, WHITE)
    put(s, -1, 0, G, WHITE)
    put(s, 0, 0, Q, BLACK)
    put(s, 1, 0, S, BLACK)
    put(s, -1, 1, B, WHITE)
    put(s, 1, -1, A, BLACK)
    put(s, -3, 1, A, WHITE)
    set_turn(s, 8)
    return s


def reserve_b3():
    s = empty_state(0)
    put(s, 0, 0, Q, BLACK)
    put(s, 1, 0, A, BLACK)
    put(s, 2, 0, Q, WHITE)
    put(s, 3, 0, A, WHITE)
    put(s, 3, -1, S, WHITE)
    put(s, 2, 1, A, WHITE)
    set_turn(s, 8)
    return s


# (builder, legal count, {immobile_only: (qualifying slots, candidate row)})
RESERVE_CASES = [
    (reserve_b1, 53, {True: ([42, 43], [42, 43, -1, -1, -1, -1, 3, 14, 25, 36, 47, 6, 17, 28, 39, 50])}),
    (reserve_b3, 55, {
        True: ([29, 40, 41, 42, 48, 50, 52], [50, 42, 48, 29, 40, 41, 3, 14, 25, 36, 47, 6, 17, 28, 39, 9]),
        False: ([29, 38, 39, 40, 41, 42, 46, 48, 50, 52, 54],
                [39, 50, 42, 48, 29, 40, 3, 14, 25, 36, 47, 6, 17, 28, 9, 20])}),
]

CANDIDATE_SHORT = dict(n=4, priors=[0.1, 0.4, 0.3, 0.2], qual=[2],
                       row=[2, -1, -1, -1, -1, -1, 1, 3, 0, 2, 4, 5, 6, 7, 8, 9])


# ---- sequential halving -----------------------------------------------------
BASE_OVERRIDE = {(4, 20): 0.1, (4, 10): 0.1, (5, 30): 0.53, (5, 31): 0.0}
Q_OVERRIDE = {(4, 20): 0.02, (4, 10): 0.02, (5, 30): 0.0, (5, 31): 0.01}


def base_of(g, s):
    return BASE_OVERRIDE.get((g, s), ((s * 37 + g * 11) % 41 - 20) / 25.0)


def q_of(r, g, s):
    return Q_OVERRIDE.get((g, s), ((s * 13 + r * 7 + g * 5) % 23 - 11) / 400.0)


def _rows(rows, k):
    return [list(r) + [-1] * (k - len(r)) for r in rows]


_K16_ROWS = [[3, 17, 40, 8, 22, 5, 31, 12, 0, 9, 26, 14, 35, 2, 19, 11], [6, 13, 6, 1], [4], [], [20, 10], [30, 31]]
_K16_CALLS = [  # (rows passed to the round, per_slot)
    (_K16_ROWS, 2),
    ([[14, 12, 5, 35, 3, 31, 26, 22], [6, 6], [4], [], [20], [31]], 4),
    ([[31, 22, 14, 12], [6], [4], [], [20], [31]], 8),
    ([[14, 12], [6], [4], [], [20], [31]], 16),
]
_K64_CALLS = [
    ([list(range(100, 132)), [7, 7, 9]], 4),
    ([[113, 106, 104, 129, 127, 125, 122, 120, 118, 116, 114, 111, 109, 107, 105, 103], [9]], 8),
    ([[125, 116, 114, 109, 107, 105, 103, 113], [9]], 16),
    ([[105, 103, 113, 125], [9]], 32),
]

# name -> (config overrides, initial rows, [(rows, per_slot, wave)], chosen)
HALVING_CASES = {
    "k16-schedule": (dict(max_num_considered_actions=16, num_simulations=128, wave_parallel=True),
                     _rows(_K16_ROWS, 16),
                     [(_rows(r, 16 >> i), ps, (2, 4, 8, 16)[i]) for i, (r, ps) in enumerate(_K16_CALLS)],
                     [14, 6, 4, 0, 20, 31]),
    "k16-w1": (dict(max_num_considered_actions=16, num_simulations=128, wave_parallel=False),
               _rows(_K16_ROWS, 16),
               [(_rows(r, 16 >> i), ps, 1) for i, (r, ps) in enumerate(_K16_CALLS)],
               [14, 6, 4, 0, 20, 31]),
    "k64-schedule": (dict(max_num_considered_actions=64, num_simulations=1024, wave_parallel=True),
                     _rows(_K64_CALLS[0][0], 64),
                     [(_rows(r, 64 >> i), ps, (2, 4, 8, 16)[i]) for i, (r, ps) in enumerate(_K64_CALLS)],
                     [113, 9]),
}


class HalvingStub:
    """run_round / child_stats stand-ins: records each round's rows, per_slot
    and wave; a slot's visits are per_slot per column holding it, per round;
    its Q is q_of(round, game, slot)."""

    def __init__(self):
        self.calls = []
        self.visits = {}

    def run_round(self, cand, per_slot, wave):
        cand = np.asarray(cand)
        self.calls.append((cand.tolist(), int(per_slot), int(wave)))
        for g, row in enumerate(cand):
            for s in row:
                if s >= 0:
                    self.visits[(g, int(s))] = self.visits.get((g, int(s)), 0) + int(per_slot)
        return int(per_slot) * cand.shape[1] * cand.shape[0]

    def child_stats(self, cand):
        cand = np.asarray(cand)
        r = len(self.calls) - 1
        v = np.zeros(cand.shape, np.int32)
        q = np.zeros(cand.shape, np.float32)
        for g, row in enumerate(cand):
            for j, s in enumerate(row):
                if s >= 0:
                    v[g, j] = self.visits[(g, int(s))]
                    q[g, j] = q_of(r, g, int(s))
        return v, q


def halving_base(B):
    base = np.full((B, 256), -1e30, np.float32)
    for g in range(B):
        for s in range(256):
            base[g, s] = base_of(g, s)
    return base
