"""The CPU oracle against golden vectors written by the reference's own engine.

Fixtures: tests/golden/golden_c{1,2,3,4}.npz, produced by
tests/golden/make_golden.py from the reference's hive_gpu/csrc/cpu_native.cpp
compiled for the host (oracle/Makefile, target ref).  Every comparison is bit-exact (features
are compared as raw float32 bit patterns).
"""
import numpy as np
import pytest

from conftest import load_golden


def test_generator_replays_reference(oracle, golden):
    """oracle.generate_positions == random play through the reference's lists."""
    states, plies = oracle.generate_positions(len(golden["states"]), int(golden["mask"]),
                                              int(golden["max_ply"]), int(golden["seed"]))
    assert np.array_equal(plies, golden["plies"])
    assert np.array_equal(states, golden["states"])


def test_legal_moves_features_bit_exact(oracle, golden):
    moves, n, feat, _ = oracle.batch_legal_features_actions(golden["states"], threads=2)
    assert np.array_equal(n, golden["n"])
    assert np.array_equal(moves, golden["moves"])  # emission order and zero padding
    assert np.array_equal(feat.view(np.uint32), golden["features"].view(np.uint32))


def test_compact_lists_ap_queen_escape(oracle, golden):
    st = golden["states"]
    for i in range(len(st)):
        m, n = oracle.fnn_feature_moves(st[i])
        assert n == golden["ncompact"][i]
        assert np.array_equal(m, golden["compact"][i])
        assert np.array_equal(oracle.articulation(st[i]), golden["ap"][i])
        assert oracle.queen_escape(st[i]) == golden["queen_escape"][i]
    qe = oracle.batch_queen_escape(st, threads=2)
    assert np.array_equal(qe, golden["queen_escape"])


@pytest.mark.parametrize("full", [False, True])
def test_successor_features(oracle, golden, full):
    got = oracle.batch_successor_features(golden["states"], golden["moves"], golden["succ_root"],
                                          golden["succ_idx"], full_list=full, threads=2)
    want = golden["succ_features_full" if full else "succ_features"]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_apply_move_children(oracle, golden):
    st, mv = golden["states"], golden["moves"]
    for k, (r, i) in enumerate(zip(golden["succ_root"][:512], golden["succ_idx"][:512])):
        assert np.array_equal(oracle.apply_move(st[r], mv[r, i]), golden["child_states"][k])


def test_lockstep_selfplay_finals(oracle):
    g = load_golden("c4")
    finals, plies = oracle.lockstep_selfplay(len(g["finals"]), 0, int(g["max_ply"]), int(g["seed"]))
    assert np.array_equal(plies, g["plies"])
    assert np.array_equal(finals, g["finals"])


def test_root_tactical_probe(oracle):
    """root_tactical_probe_batch (game_logic.cu:290-397) on positions sampled by
    outcome (no tactic, immediate win, two-move forced win, screened list,
    forced random move, no gate), for four combinations of the enable flags."""
    g = load_golden("probe")
    kinds = set(g["kinds"].tolist())
    assert {"none", "screened", "w1", "w2", "forced", "ungated"} <= kinds
    for j, (f1, f2, f3) in enumerate(g["flags"]):
        win, allowed, forced = oracle.batch_root_tactical_probe(g["states"], g["legal"], g["nlegal"], g["priors"],
                                                                f1, f2, f3, threads=2)
        assert np.array_equal(win, g["win"][j]), (f1, f2, f3)
        assert np.array_equal(allowed, g["allowed"][j]), (f1, f2, f3)
        assert np.array_equal(forced, g["forced"][j]), (f1, f2, f3)
    kids = g["child_states"]
    got = np.array([oracle.immediate_win(kids[i]) for i in range(len(kids))], np.uint8)
    assert np.array_equal(got, g["child_immediate_win"])
    assert got.any() and not got.all()
