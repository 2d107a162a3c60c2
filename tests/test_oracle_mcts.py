"""Pins of the MCTS tree oracle (oracle/hive_mcts_oracle.c): invariants the
reference's tree kernels guarantee (mcts_tree.cuh:689-1234) and hand-built
trees with known answers.  No reference test pins these kernels."""
import numpy as np
import pytest

from mcts_driver import OracleEngine, run_search
from oracle.mcts import MctsOracle, new_tree


@pytest.fixture(scope="module")
def roots(oracle):
    st, _ = oracle.generate_positions(12, 7, 40, 0xC0FFEE)
    return st


def _check_counts(t, records):
    """N(node) = simulations ending at node + sum of children's N; no outstanding virtual loss."""
    B, M = t["visit_count"].shape
    ended = np.zeros((B, M), np.int64)
    for r in records[1:]:
        for s, leaf in enumerate(r["leaf"]):
            if leaf >= 0:
                ended[s % B, leaf] += 1
    vc, fc, nc = t["visit_count"], t["first_child"], t["num_children"]
    for g in range(B):
        for u in range(int(t["node_count"][g])):
            kids = vc[g, fc[g, u]: fc[g, u] + nc[g, u]].sum() if fc[g, u] >= 0 else 0
            assert vc[g, u] == ended[g, u] + kids, (g, u)
            assert abs(float(t["total_value"][g, u])) <= vc[g, u] + 1e-4
    assert not t["virtual_q_penalty"].any()


@pytest.mark.parametrize("mode,W", [("slots", 1), ("slots", 2), ("mask", 3)])
def test_search_invariants(roots, mode, W):
    t, rec = run_search(OracleEngine(), roots, W=W, mode=mode, waves=5)
    _check_counts(t, rec)
    B = roots.shape[0]
    # node pool accounting: 1 + children of every expanded node
    for g in range(B):
        expanded = t["first_child"][g] >= 0
        assert t["node_count"][g] == 1 + t["num_children"][g][expanded].sum()
    # mid-wave: each selection adds one virtual visit to every node it entered
    for before, r in zip(rec[:-1], rec[1:]):
        entered = np.zeros_like(r["mid_visits"])
        for s in range(r["leaf"].shape[0]):
            for k in range(r["vlen"][s]):
                entered[s % B, r["vl"][s, k]] += 1
        assert np.array_equal(r["mid_visits"] - before["post_visits"], entered)


def test_children_in_legal_order(oracle, roots):
    t, rec = run_search(OracleEngine(), roots, W=2, waves=4)
    for g in range(roots.shape[0]):
        if t["first_child"][g, 0] < 0:
            continue
        moves, n = oracle.legal_moves(roots[g])
        f = t["first_child"][g, 0]
        assert t["num_children"][g, 0] == n
        assert np.array_equal(t["move_bytes"][g, f:f + n], moves[:n])
        assert (t["parent_idx"][g, f:f + n] == 0).all()
        cq, cr = oracle.centroid(roots[g])
        assert [oracle.move_to_action(moves[i], cq, cr) for i in range(n)] == list(t["action_idx"][g, f:f + n])


def _tiny_tree(priors, M=16):
    t = new_tree(1, M)
    n = len(priors)
    t["first_child"][0, 0] = 1
    t["num_children"][0, 0] = n
    t["node_count"][0] = 1 + n
    t["prior"][0, 1:1 + n] = priors
    t["parent_idx"][0, 1:1 + n] = 0
    for i in range(n):
        t["move_bytes"][0, 1 + i] = [2, 0, 0, 0, 0, 0]  # PASS moves
    return t


def test_puct_known_answers_and_sign_alternation(oracle):
    m = MctsOracle(oracle)
    t = _tiny_tree([0.1, 0.6, 0.3])
    alive = np.zeros((1, 256), np.int8)
    alive[0, :3] = 1
    # an unvisited root has sqrt(N)=0: every score is 0 and the first child wins
    leaf, _, _, _, _ = m.select_mask(t, np.ones(1, np.int8), np.zeros(1, np.int32), alive, 1.25, 1)
    assert leaf[0] == 1
    t = _tiny_tree([0.1, 0.6, 0.3])
    t["visit_count"][0, 0] = 1
    leaf, paths, plen, vl, vlen = m.select_mask(t, np.ones(1, np.int8), np.zeros(1, np.int32), alive, 1.25, 1)
    assert leaf[0] == 2 and plen[0] == 1 and vl[0, 0] == 2  # max prior wins with no child visits
    assert t["visit_count"][0, 2] == 1 and t["total_value"][0, 2] == -1.0  # virtual loss
    st = oracle.init_state(0)
    leaves = np.repeat(st[None], 1, axis=0)
    legal, nl = oracle.legal_moves(st)
    z = np.zeros((1, 256), np.float32)
    m.expand_backprop_dense(t, z, leaf, leaves, legal[None], np.array([0], np.int32), z, np.zeros(1, np.int32),
                            np.array([0.5], np.float32), vl, vlen)
    # the leaf was not expanded (n=0 given), so 0.0 is backed up; virtual loss undone
    assert t["visit_count"][0, 2] == 1 and t["total_value"][0, 2] == 0.0
    assert t["visit_count"][0, 0] == 2
    # second simulation: child 2 now has N=1, W=0 -> q=0; PUCT favours child 3 (prior 0.3) over 2?
    leaf2, _, _, vl2, vlen2 = m.select_mask(t, np.ones(1, np.int8), np.zeros(1, np.int32), alive, 1.25, 1)
    # scores: c2: 0 + (1.25*0.6)*sqrt2/2 ; c3: (1.25*0.3)*sqrt2/1 -- equal in float32; first wins (node 2)
    assert leaf2[0] == 2
    # expanding sim with value v: W(leaf) = v, W(parent) = -v (sign alternation)
    legal, nl = oracle.legal_moves(st)
    pri = np.zeros((1, 256), np.float32)
    pri[0, :nl] = 1.0 / nl
    m.expand_backprop_dense(t, z, leaf2, leaves, legal[None], np.array([nl], np.int32), pri,
                            np.zeros(1, np.int32), np.array([0.5], np.float32), vl2, vlen2)
    assert t["num_children"][0, 2] == nl and t["first_child"][0, 2] == 4
    assert t["total_value"][0, 2] == 0.5 and t["total_value"][0, 0] == -0.5
    assert t["node_count"][0] == 4 + nl


def test_terminal_and_pool_exhaustion(oracle):
    m = MctsOracle(oracle)
    t = _tiny_tree([0.5, 0.5], M=5)
    t["visit_count"][0, 0] = 1
    alive = np.zeros((1, 256), np.int8)
    alive[0, :2] = 1
    leaf, _, _, vl, vlen = m.select_mask(t, np.ones(1, np.int8), np.zeros(1, np.int32), alive, 1.0, 1)
    st = oracle.init_state(0)
    legal, nl = oracle.legal_moves(st)  # 4 placements > 2 free slots: the pool cannot take them
    pri = np.full((1, 256), 0.25, np.float32)
    z = np.zeros((1, 256), np.float32)
    m.expand_backprop_dense(t, z, leaf, st[None], legal[None], np.array([nl], np.int32), pri,
                            np.zeros(1, np.int32), np.array([0.9], np.float32), vl, vlen)
    assert t["first_child"][0, leaf[0]] == -1 and t["node_count"][0] == 3
    assert t["total_value"][0, leaf[0]] == 0.0  # not expanded: 0.0 backed up
    # terminal leaf: white to move (turn even) after white won -> +1 for the leaf's player
    leaf, _, _, vl, vlen = m.select_mask(t, np.ones(1, np.int8), np.zeros(1, np.int32), alive, 1.0, 1)
    won = st.copy()
    won[3415] = 1
    m.expand_backprop_dense(t, z, leaf, won[None], legal[None], np.array([nl], np.int32), pri,
                            np.ones(1, np.int32), np.array([0.9], np.float32), vl, vlen)
    assert t["is_terminal"][0, leaf[0]] == 1 and t["terminal_value"][0, leaf[0]] == 1.0
    assert t["total_value"][0, leaf[0]] == 1.0


# ---- legacy action-space engine (mcts_tree.cuh:205-687) -------------------------------------
@pytest.mark.parametrize("split", [False, True])
def test_legacy_search_invariants(oracle, roots, split):
    """Visit conservation and no outstanding virtual loss after waves of the legacy
    loop; children = the legal moves with an action index, in list order, with
    their action-space priors; the fused and split backups agree."""
    from mcts_driver import run_search_legacy
    t, rec, pols = run_search_legacy(OracleEngine(), roots, W=2, waves=4, split=split)
    _check_counts(t, rec)
    B = roots.shape[0]
    for g in range(B):
        expanded = t["first_child"][g] >= 0
        assert t["node_count"][g] == 1 + t["num_children"][g][expanded].sum()
    t2, _, pols2 = run_search_legacy(OracleEngine(), roots, W=2, waves=4, split=not split)
    for k in t:
        assert np.array_equal(t[k], t2[k]), k
    for g in range(B):
        f = t["first_child"][g, 0]
        if f < 0:
            continue
        moves, n = oracle.legal_moves(roots[g])
        cq, cr = oracle.centroid(roots[g])
        acts = [oracle.move_to_action(moves[i], cq, cr) for i in range(n)]
        keep = [i for i in range(n) if acts[i] >= 0]
        assert t["num_children"][g, 0] == len(keep)
        assert np.array_equal(t["move_bytes"][g, f:f + len(keep)], moves[keep])
        assert list(t["action_idx"][g, f:f + len(keep)]) == [acts[i] for i in keep]


def test_legacy_policy_known_answers(oracle, roots):
    """extract_policy: visit distribution at temperature 1, pruning below 20% of
    the maximum, visits^2 at temperature 0.5, one-hot argmax past the drop move."""
    from mcts_driver import run_search_legacy
    t, _, (p1, pp, p05) = run_search_legacy(OracleEngine(), roots, W=2, waves=4)
    B = roots.shape[0]
    for g in range(B):
        f, n = t["first_child"][g, 0], t["num_children"][g, 0]
        if f < 0 or n == 0:
            assert not p1[g].any()
            continue
        v = t["visit_count"][g, f:f + n].astype(np.float64)
        a = t["action_idx"][g, f:f + n]
        if g % 3 == 2:  # move number 20 >= 15: greedy
            want = np.zeros(85834)
            want[a[int(np.argmax(v))]] = 1.0
            assert np.array_equal(p1[g], want) and np.array_equal(p05[g], want)
            continue
        np.testing.assert_allclose(p1[g][a], v / v.sum(), rtol=1e-6)
        assert abs(p1[g].sum() - 1.0) < 1e-5
        pv = np.where(v < v.max() * 0.2, 0.0, v)
        np.testing.assert_allclose(pp[g][a], pv / pv.sum(), rtol=1e-6)
        np.testing.assert_allclose(p05[g][a], v ** 2 / (v ** 2).sum(), rtol=1e-5)


def test_legacy_select_first_child_fallback():
    """A node whose children all score -1e30 or below descends to its first child."""
    m = MctsOracle()
    t = new_tree(1, 16)
    t["first_child"][0, 0], t["num_children"][0, 0] = 1, 3
    t["parent_idx"][0, 1:4] = 0
    t["node_count"][0] = 4
    t["virtual_q_penalty"][0, 1:4] = 1e31  # q - penalty far below -1e30
    leaf, paths, plen, vl, vlen = m.select_legacy(t, np.ones(1, np.int8), np.zeros(1, np.int32), 1.25, 1)
    assert leaf[0] == 1 and plen[0] == 1 and list(vl[0, :1]) == [1]


def test_legal_mask_is_action_scatter(oracle, roots):
    m = MctsOracle()
    legal, n, _, act = oracle.batch_legal_features_actions(roots)
    mask = m.legal_mask(roots, legal, n)
    for g in range(roots.shape[0]):
        want = np.zeros(85834, np.float32)
        a = act[g, :n[g]]
        want[a[a >= 0]] = 1.0
        assert np.array_equal(mask[g], want)


@pytest.mark.parametrize("mode", ["slots", "mask"])
def test_completed_q_descent_known_answers(oracle, mode):
    """deterministic_non_root descent (mcts_tree.cuh:77-143) on hand-built
    trees whose choice was computed by hand in float64 (tests/mcts_driver.py
    COMPLETED_Q_CASES: each plausible misreading of the rule picks another child)."""
    from mcts_driver import COMPLETED_Q_CASES, completed_q_trees
    t, want = completed_q_trees()
    B = want.shape[0]
    m = MctsOracle(oracle)
    if mode == "slots":
        leaf, paths, plen, vl, vlen = m.select_slots(t, np.ones(B, np.int8), np.zeros(B, np.int32),
                                                     np.zeros((B, 1), np.int32), 256, 1.25, 1, True, 4.0, 0.0)
    else:
        leaf, paths, plen, vl, vlen = m.select_mask(t, np.ones(B, np.int8), np.zeros(B, np.int32),
                                                    np.ones((B, 1), np.int8), 1.25, 1, True, 4.0, 0.0)
    assert np.array_equal(leaf, want)
    # the chosen child takes N + 1; a forced root child (slots) takes no virtual
    # loss in this mode (mcts_tree.cuh:879-885), one chosen by the mask does
    assert (plen == 2).all() and np.array_equal(vl[np.arange(B), vlen - 1], want)
    assert (vlen == (1 if mode == "slots" else 2)).all()
    assert np.array_equal(t["visit_count"][np.arange(B), want], [c[0][w - 2][0] + 1 for c, w in
                                                                 zip(COMPLETED_Q_CASES, want)])


@pytest.mark.parametrize("eps,temp,pad", __import__("mcts_driver").NOISE_CASES)
def test_root_noise_known_answers(eps, temp, pad):
    """or_mcts_root_noise (mcts_tree.cuh:1192-1234) against the float64 closed form
    of tests/mcts_driver.py (NOISE_CASES).  Tolerance 2 float32 ulp: at T = 2 the
    roots and their sum are exact, then one division and the two roundings of the
    mix; with eps = 0 and T <= 1 the priors must come back bit for bit."""
    from mcts_driver import OracleEngine, check_noise_case
    got = check_noise_case(OracleEngine(), eps, temp, pad, ulps=2.0)
    if eps == 0.0 and temp <= 1.0:
        assert np.array_equal(got["prior"][0, 1:5], np.array(__import__("mcts_driver").NOISE_PRIORS, np.float32))


def test_root_noise_cases_discriminate():
    """Each misreading the closed form rules out moves a prior by far more than 2 ulp
    (the tolerance above), so the known answers pin the order and the terms."""
    from mcts_driver import NOISE_PRIORS, NOISE_ROW, noise_expected
    p = np.array(NOISE_PRIORS)
    z = np.array(NOISE_ROW, np.float32).astype(np.float64)
    r = np.sqrt(p) / np.sqrt(p).sum()
    right = noise_expected(0.25, 2.0, 4)
    wrong = {
        "eps on the prior": 0.25 * r + 0.75 * z,
        "mix before temperature": np.sqrt(0.75 * p + 0.25 * z) / np.sqrt(0.75 * p + 0.25 * z).sum(),
        "p^T": 0.75 * (p ** 2 / (p ** 2).sum()) + 0.25 * z,
        "no renormalisation": 0.75 * np.sqrt(p) + 0.25 * z,
    }
    for name, w in wrong.items():
        assert np.abs(w - right).max() > 1e-3, name
    assert np.abs(noise_expected(0.25, 0.5, 4) - noise_expected(0.25, 1.0, 4)).max() == 0.0
    assert np.abs(noise_expected(0.25, 2.0, 2)[2:] - r[2:]).max() == 0.0


@pytest.mark.parametrize("mode", ["slots", "mask"])
def test_q_penalty_known_answers(oracle, mode):
    """deterministic_non_root with q_penalty 0.25 (mcts_tree.cuh:770-777,929-934 in the
    selects, :1164-1172 in the backup) on the hand-worked tree of tests/mcts_driver.py:
    the penalty turns the second simulation away from node 2, selection leaves N + 1 and
    vq + 0.25 on the nodes it entered, the backup takes the penalty off again and keeps
    the selection's N + 1 (in root-mask mode the root child's ordinary virtual loss stays
    and its vq ends at -0.25)."""
    from mcts_driver import OracleEngine, check_q_penalty_case
    check_q_penalty_case(OracleEngine(), oracle.init_state(0), mode)
