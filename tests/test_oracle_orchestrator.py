"""Known answers for the numpy restatement of the orchestrator's host logic
(oracle/orchestrator.py), on the CPU.

The reference has no test of its orchestrator (fnn_mcts_orchestrator.py), so
the restatement's pieces are pinned here by what the mathematics or the
reference's own primitives fix: the policy-target temperature search against
its closed form, stable top-k tie order, immediate wins against the
reference's win detector (golden probe vectors), and queen-surround counts
against the C oracle's independent count.
"""
import math

import numpy as np
import pytest

from conftest import load_golden


def _cfg(**kw):
    from hive_neuralnet_amd.orchestrator import FNNMCTSConfig
    return FNNMCTSConfig(**kw)


def test_policy_target_uniform_and_masked():
    from oracle.orchestrator import policy_target
    cfg = _cfg(adaptive_policy_target_temperature=False, policy_target_temperature=2.0)
    sampled = np.zeros((3, 256), np.float32)
    valid = np.zeros((3, 256), bool)
    for g, n in enumerate((1, 5, 256)):
        valid[g, :n] = True
    p, t = policy_target(cfg, sampled, valid)
    assert np.allclose(t, 2.0)
    for g, n in enumerate((1, 5, 256)):
        assert np.allclose(p[g, :n], 1.0 / n, rtol=1e-6) and not p[g, n:].any()


@pytest.mark.parametrize("a,cap", [(3.0, 0.7), (5.0, 0.6), (1.0, 0.7)])
def test_policy_target_adaptive_temperature_closed_form(a, cap):
    """Two legal slots with logits (a, 0): the top-1 probability at
    temperature T is 1 / (1 + exp(-a / T)), so the capped temperature is
    T* = a / ln(cap / (1 - cap)); the 12-step bisection over [1, 7] returns
    the upper end of its last bracket, within 6 / 4096 above T* (7 when T*
    is beyond the range).  When the base temperature already meets the cap
    it is returned unchanged."""
    from oracle.orchestrator import policy_target
    cfg = _cfg(policy_target_top1_cap=cap, policy_target_min_temperature=1.0, policy_target_max_temperature=7.0)
    sampled = np.full((1, 256), -1e30, np.float32)
    sampled[0, 0], sampled[0, 1] = a, 0.0
    valid = np.zeros((1, 256), bool)
    valid[0, :2] = True
    p, t = policy_target(cfg, sampled, valid)
    t_star = a / math.log(cap / (1.0 - cap))
    if 1.0 / (1.0 + math.exp(-a)) <= cap:
        assert t[0] == 1.0
    elif t_star >= 7.0:  # the cap is out of reach: the search ends at the maximum temperature
        assert t[0] == 7.0
    else:
        assert t_star - 1e-5 <= t[0] <= t_star + 6.0 / 4096 + 1e-5
        assert p[0, 0] <= cap + 1e-6
    assert abs(float(p[0, :2].sum()) - 1.0) < 1e-6 and not p[0, 2:].any()


def test_stable_topk_ties_lowest_slot():
    from oracle.orchestrator import _stable_topk
    x = np.array([[0.5, 1.0, 1.0, 0.2, 1.0, 0.5]], np.float32)
    assert _stable_topk(x, 4).tolist() == [[1, 2, 4, 0]]


def test_immediate_wins_match_reference_detector(oracle):
    """SearchPlyOracle.immediate_wins (first winning slot, :446-493) finds a
    win exactly in the roots the reference's probe vectors mark as
    win-in-one ("w1") and in the child positions whose reference detector
    (has_immediate_surround_win_for_current_player) fires; the slot it
    returns wins for the mover and no lower slot does."""
    from oracle.orchestrator import SearchPlyOracle
    g = load_golden("probe")
    s = SearchPlyOracle(_cfg())
    kinds = g["kinds"]
    sel = np.concatenate([np.nonzero(kinds == k)[0][:6] for k in sorted(set(kinds.tolist()))])
    st, lm, n = g["states"][sel], g["legal"][sel], g["nlegal"][sel]
    wins = s.immediate_wins(st, lm, n)
    assert np.array_equal(wins >= 0, kinds[sel] == "w1")
    for i in np.nonzero(wins >= 0)[0]:
        white = (int(st[i, 3412]) | (int(st[i, 3413]) << 8)) % 2 == 0
        res = [int(oracle.apply_move(st[i], lm[i, j])[3415]) for j in range(int(wins[i]) + 1)]
        mover = [(r == 1 and white) or (r == 2 and not white) for r in res]
        assert mover[-1] and not any(mover[:-1])
    cs, cw = g["child_states"][:120], g["child_immediate_win"][:120]
    clm, cn, _, _ = oracle.batch_legal_features_actions(cs, want_features=False, want_actions=False)
    assert np.array_equal(s.immediate_wins(cs, clm, cn) >= 0, cw != 0)


def test_surround_counts_match_c_oracle(oracle):
    """The restatement's queen-surround count (used by the reserve-slot rule,
    :339-382) against the C oracle's own count on golden positions."""
    from oracle.orchestrator import _surround
    for name in ("c2", "c3"):
        st = load_golden(name)["states"][:64]
        for s in st:
            for colour in (0, 1):
                assert _surround(s, colour) == oracle.surround_count(s, colour)


@pytest.mark.parametrize("name", ["k16-schedule", "k16-w1", "k64-schedule"])
def test_sequential_halving_known_answers(name):
    """oracle.orchestrator.sequential_halving against the hand-worked cases
    of tests/orchestrator_cases.py: the rows of every round, per_slot, the
    wave width and the final choice."""
    from orchestrator_cases import HALVING_CASES, HalvingStub, halving_base
    from oracle.orchestrator import sequential_halving
    over, rows, calls, chosen = HALVING_CASES[name]
    cand = np.array(rows, np.int32)
    stub = HalvingStub()
    got = sequential_halving(_cfg(**over), cand, halving_base(cand.shape[0]), stub.run_round, stub.child_stats)
    assert stub.calls == calls
    assert got.tolist() == chosen


@pytest.mark.parametrize("case", [0, 1])
def test_reserve_candidates_known_answers(oracle, case):
    """The queen-surround reserve rule (fnn_mcts_orchestrator.py:339-444) on
    hand-built positions: which moves qualify, with and without the
    immobile-queen filter, and the candidate row they give with the
    tests/orchestrator_cases.py priors."""
    from orchestrator_cases import RESERVE_CASES, priors_formula
    from oracle.orchestrator import SearchPlyOracle, candidate_row
    build, n, want = RESERVE_CASES[case]
    s = build()[None]
    legal, nl = oracle.legal_moves(s[0])
    assert nl == n
    for immobile, (qual_slots, row) in want.items():
        ref = SearchPlyOracle(_cfg(queen_surround_reserve_immobile_only=immobile))
        qual = ref.qualifying(s, legal[None], np.array([n]))
        assert np.nonzero(qual[0])[0].tolist() == qual_slots
        valid = (np.arange(256) < n)[None]
        assert candidate_row(qual, valid, priors_formula(n)[None], 16, 6)[0].tolist() == row


def test_candidate_row_short_list():
    """Fewer legal moves than fill columns: the fill continues with the
    reserve slot (lowest slot first among the -1e30 entries), then illegal slots."""
    from orchestrator_cases import CANDIDATE_SHORT as c
    from oracle.orchestrator import candidate_row
    priors = np.zeros((1, 256), np.float32)
    priors[0, :c["n"]] = c["priors"]
    qual = np.zeros((1, 256), bool)
    qual[0, c["qual"]] = True
    valid = (np.arange(256) < c["n"])[None]
    assert candidate_row(qual, valid, priors, 16, 6)[0].tolist() == c["row"]
