"""GPU MCTS tree kernels (through the C-ABI) against the tree oracle.

The same seeded search (tests/mcts_driver.py: root expansion, root noise,
waves of select / replay / legal / expand + backup with recorded synthetic
network outputs) runs on the oracle and on the GPU; every tree array,
selection output and leaf state must be bit-identical.
"""
import numpy as np
import pytest

from mcts_driver import GpuEngine, OracleEngine, run_search, synthetic_eval, tree_equal

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def roots(oracle):
    st, _ = oracle.generate_positions(48, 7, 60, 0xC0FFEE)
    return st


@pytest.mark.parametrize("mode,W,C,M,dup", [("slots", 1, 4, 8192, False), ("slots", 2, 4, 8192, False),
                                            ("slots", 4, 2, 8192, False), ("mask", 3, 4, 8192, False),
                                            ("slots", 2, 4, 300, False), ("slots", 3, 16, 8192, False),
                                            ("slots", 2, 4, 8192, True)],
                         ids=["slots-w1", "slots-w2", "slots-w4", "mask-w3", "slots-pool-exhaustion", "slots-c16-w3",
                              "slots-duplicate"])
def test_search_matches_oracle(roots, mode, W, C, M, dup):
    ot, orec = run_search(OracleEngine(), roots, W=W, C=C, M=M, mode=mode, waves=6, dup=dup)
    gt, grec = run_search(GpuEngine(), roots, W=W, C=C, M=M, mode=mode, waves=6, dup=dup)
    assert tree_equal(ot, gt) == []
    assert np.array_equal(orec[0]["was_root"], grec[0]["was_root"])
    for a, b in zip(orec[1:], grec[1:]):
        for k in ("leaf", "paths", "plen", "vl", "vlen", "leaves", "mid_visits"):
            assert np.array_equal(a[k], b[k]), k
        assert np.array_equal(a["mid_total"].view(np.uint32), b["mid_total"].view(np.uint32))


@pytest.mark.parametrize("mode,W,qp", [("slots", 2, 0.25), ("slots", 1, 0.0), ("mask", 3, 0.25)],
                         ids=["slots-w2-penalty", "slots-w1", "mask-w3-penalty"])
def test_search_completed_q_matches_oracle(roots, mode, W, qp):
    """deterministic_non_root: completed-Q descent below the root, the q
    penalty as virtual loss (W > 1) and its undo in the backup."""
    kw = dict(W=W, C=4, M=8192, mode=mode, waves=6, det=True, sigma=4.0, qp=qp)
    ot, orec = run_search(OracleEngine(), roots, **kw)
    gt, grec = run_search(GpuEngine(), roots, **kw)
    assert tree_equal(ot, gt) == []
    for a, b in zip(orec[1:], grec[1:]):
        for k in ("leaf", "paths", "plen", "vl", "vlen", "leaves", "mid_visits"):
            assert np.array_equal(a[k], b[k]), k
        assert np.array_equal(a["mid_total"].view(np.uint32), b["mid_total"].view(np.uint32))


def test_fused_select_replay_legal_fnn(roots):
    import torch
    eng = GpuEngine()
    ext = eng.ext
    B = roots.shape[0]
    t = eng.tree(B, 4096)
    legal, n = eng.legal(roots)
    pri = np.zeros((B, 256), np.float32)
    for i in range(B):
        pri[i, : n[i]] = 1.0 / max(1, n[i])
    z = np.zeros((B, 256), np.float32)
    res = roots[:, 3415].astype(np.int32)
    leaf0 = np.where(res == 0, 0, -1).astype(np.int32)
    eng.expand_dense(t, z, leaf0, roots, legal, n, pri, res)
    slots = np.tile(np.arange(4, dtype=np.int32), (B, 1))
    slots[n[:, None] <= np.arange(4)[None, :]] = -1
    out = ext.mcts_select_replay_legal_fnn_root_slots_batch(
        *eng.args(t), t["child_init_q"], eng.c(roots), eng.c((res == 0).astype(np.int8)), t["root_node"],
        eng.c(slots), 4, 256, 1.25, B, 2, 4096)
    leaf_idx, leaf_states, moves, nl, feat, results, vl, vlen = out
    assert leaf_states.shape == (8 * B, 3424) and feat.shape == (8 * B, 122)
    from oracle import Oracle
    o = Oracle()
    ls = leaf_states.cpu().numpy()
    om, on, of, _ = o.batch_legal_features_actions(ls)
    assert np.array_equal(nl.cpu().numpy(), on)
    assert np.array_equal(moves.cpu().numpy(), om)
    assert np.array_equal(feat.cpu().numpy().view(np.uint32), of.view(np.uint32))
    inactive = leaf_idx.cpu().numpy() < 0
    assert (ls[inactive] == 0).all()  # skipped rows stay all-zero states
    assert torch.equal(results, leaf_states[:, 3415].to(torch.int32))


@pytest.mark.parametrize("split", [False, True], ids=["fused", "split"])
def test_legacy_engine_matches_oracle(roots, split):
    """The legacy action-space entry points (select / expand / backprop /
    expand + backprop / extract policy) against the tree oracle: trees,
    selections, leaves, expansion flags and policies.  Policies at
    temperature 1 are bit-exact; at temperature 0.5 they go through powf,
    whose device and host implementations may differ in the last place."""
    from mcts_driver import run_search_legacy
    ot, orec, opol = run_search_legacy(OracleEngine(), roots[:24], W=2, waves=4, split=split)
    gt, grec, gpol = run_search_legacy(GpuEngine(), roots[:24], W=2, waves=4, split=split)
    assert tree_equal(ot, gt) == []
    assert np.array_equal(orec[0]["was_root"], grec[0]["was_root"])
    for a, b in zip(orec[1:], grec[1:]):
        for k in ("leaf", "paths", "plen", "vl", "vlen", "leaves") + (("was",) if split else ()):
            assert np.array_equal(a[k], b[k]), k
    assert np.array_equal(opol[0].view(np.uint32), gpol[0].view(np.uint32))
    assert np.array_equal(opol[1].view(np.uint32), gpol[1].view(np.uint32))
    np.testing.assert_allclose(gpol[2], opol[2], rtol=2e-7, atol=0)


def test_legal_mask_matches_oracle(roots):
    ge, oe = GpuEngine(), OracleEngine()
    gm, gn = ge.legal_mask(roots)
    om, on = oe.legal_mask(roots)
    assert np.array_equal(gn, on)
    assert np.array_equal(gm.view(np.uint32), om.view(np.uint32))
    moves, n, masks = ge.ext.generate_legal_moves_and_mask_batch(ge.c(roots), roots.shape[0])
    assert np.array_equal(masks.cpu().numpy(), gm) and np.array_equal(n.cpu().numpy(), on)


@pytest.mark.parametrize("total", [1, 1000, 5000])
def test_wave_stats(total):
    """hg_mcts_wave_stats accumulates (leaves reached, their legal counts,
    their virtual-loss lengths, rows) in stream order over several calls."""
    import torch
    from hive_neuralnet_amd import hive_gpu
    ext = hive_gpu.load_extension()
    rng = np.random.default_rng(total)
    stats = torch.zeros((4,), dtype=torch.int64, device="cuda")
    want = np.zeros(4, np.int64)
    for _ in range(3):
        leaf = rng.integers(-1, 50, size=total).astype(np.int32)
        nl = rng.integers(0, 257, size=total).astype(np.int32)
        vl = rng.integers(0, 64, size=total).astype(np.int32)
        ext.mcts_wave_stats(torch.from_numpy(leaf).cuda(), torch.from_numpy(nl).cuda(), torch.from_numpy(vl).cuda(),
                            total, stats)
        live = leaf >= 0
        want += (live.sum(), nl[live].sum(), vl[live].sum(), total)
    assert np.array_equal(stats.cpu().numpy(), want)


def test_replay_fill_writes_idle_rows(roots):
    """hg_mcts_replay_fill over a buffer of stale bytes: replayed rows as
    hg_mcts_replay, rows of idle simulations (leaf index < 0) all zero."""
    import torch
    ge, oe = GpuEngine(), OracleEngine()
    B = roots.shape[0]
    T = 3 * B
    rng = np.random.default_rng(5)
    t = oe.tree(B, 4096)
    legal, n = oe.legal(roots)
    pri, _, cq = synthetic_eval(rng, n, B)
    res = roots[:, 3415].astype(np.int32)
    act = (res == 0) & (n > 0)
    oe.expand_dense(t, cq, np.where(act, 0, -1).astype(np.int32), roots, legal, n, pri, res)
    slots = np.where(n[:, None] > np.arange(3)[None, :], np.arange(3)[None, :], -1).astype(np.int32)
    idle = act.copy()
    idle[::4] = False  # every fourth game idle: its simulations are empty
    leaf, paths, plen, _, _ = oe.select_slots(t, idle, slots, 256, 1.25, 1)
    assert (leaf < 0).any() and (leaf >= 0).any()
    want = oe.replay(roots, paths, plen, leaf)
    buf = torch.full((T, 3424), 0xAB, dtype=torch.uint8, device="cuda")
    ge.ext.mcts_replay_fill_batch(ge.c(roots), buf, ge.c(paths), ge.c(plen), ge.c(leaf), B, T)
    assert np.array_equal(buf.cpu().numpy(), want)


@pytest.mark.parametrize("mode", ["slots", "mask"])
def test_completed_q_descent_known_answers(mode):
    """The deterministic_non_root descent on the GPU against hand-computed
    float64 choices (tests/mcts_driver.py COMPLETED_Q_CASES, mcts_tree.cuh:77-143)."""
    import torch
    from mcts_driver import COMPLETED_Q_CASES, completed_q_trees
    eng = GpuEngine()
    t0, want = completed_q_trees()
    t = {k: eng.c(v) for k, v in t0.items()}
    B = want.shape[0]
    active = torch.ones((B,), dtype=torch.int8, device="cuda")
    if mode == "slots":
        out = eng.ext.mcts_select_with_root_slots_batch(
            *eng.args(t), t["child_init_q"], active, t["root_node"], torch.zeros((B, 1), dtype=torch.int32,
                                                                               device="cuda"),
            1, 256, 1.25, B, 1, eng.M(t), True, 4.0, 0.0)
    else:
        out = eng.ext.mcts_select_with_root_mask_batch(
            *eng.args(t), t["child_init_q"], active, t["root_node"], torch.ones((B, 1), dtype=torch.int8,
                                                                              device="cuda"),
            1, 1.25, B, 1, eng.M(t), True, 4.0, 0.0)
    leaf, paths, plen, vl, vlen = [o.cpu().numpy() for o in out]
    assert np.array_equal(leaf, want)
    vc = t["visit_count"].cpu().numpy()
    assert np.array_equal(vc[np.arange(B), want], [c[0][w - 2][0] + 1 for c, w in zip(COMPLETED_Q_CASES, want)])
    assert (plen == 2).all() and np.array_equal(vl[np.arange(B), vlen - 1], want)


class _OneWavePerGame(GpuEngine):
    """GpuEngine whose expansion + backup calls the original one-wave-per-game
    entry (hg_mcts_expand_backprop_dense) through the C-ABI."""

    def expand_backprop(self, t, cq, leaf, states, legal, n, pri, results, vals, vl, vlen, qp=0.0):
        import ctypes
        import torch
        from hive_neuralnet_amd.hive_gpu import _tree_struct
        B, M = t["node_count"].shape[0], self.M(t)
        tree = _tree_struct(self.args(t), t["child_init_q"], B, M)
        ins = [self.c(x) for x in (cq, leaf, states, legal, n, pri, results, vals, vl, vlen)]
        err = self.ext._lib.hg_mcts_expand_backprop_dense(ctypes.byref(tree), *[x.data_ptr() for x in ins],
                                                          float(qp), B, leaf.shape[0],
                                                          torch.cuda.current_stream().cuda_stream)
        assert err == 0
        torch.cuda.synchronize()


@pytest.mark.parametrize("mode,W,C,M,dup,det,qp", [
    ("slots", 2, 16, 8192, False, False, 0.0), ("slots", 4, 4, 8192, True, False, 0.0),
    ("slots", 3, 4, 700, False, False, 0.0), ("slots", 2, 4, 8192, False, True, 0.25),
    ("slots", 1, 4, 8192, False, True, 0.0), ("mask", 3, 4, 8192, False, False, 0.0)],
    ids=["c16-w2", "duplicate-w4", "pool-short", "completed-q-w2", "completed-q-w1", "mask-w3"])
def test_parallel_expand_backprop_equals_one_wave(roots, mode, W, C, M, dup, det, qp):
    """hg_mcts_expand_backprop_dense_ws (root children in parallel after a
    planning launch; the Python binding's path) against the original entry:
    identical trees and selections after every wave, including duplicate
    candidate slots (one root child, two columns), a node pool that runs short
    (those games take the one-wave order), completed-Q descent with and
    without the q penalty, and root-mask selection."""
    kw = dict(W=W, C=C, M=M, mode=mode, waves=6, dup=dup, det=det, sigma=4.0, qp=qp)
    a_t, a_rec = run_search(GpuEngine(), roots, **kw)
    b_t, b_rec = run_search(_OneWavePerGame(), roots, **kw)
    assert tree_equal(a_t, b_t) == []
    for a, b in zip(a_rec[1:], b_rec[1:]):
        for k in ("leaf", "paths", "plen", "vl", "vlen", "mid_visits"):
            assert np.array_equal(a[k], b[k]), k
        assert np.array_equal(a["mid_total"].view(np.uint32), b["mid_total"].view(np.uint32))


@pytest.mark.parametrize("eps,temp,pad", __import__("mcts_driver").NOISE_CASES)
def test_root_noise_known_answers(eps, temp, pad):
    """k_root_noise against the float64 closed form (tests/mcts_driver.py NOISE_CASES),
    within 2 float32 ulp (as the oracle); untouched priors and arrays bit for bit."""
    from mcts_driver import check_noise_case
    check_noise_case(GpuEngine(), eps, temp, pad, ulps=2.0)


def test_root_noise_temperature_matches_oracle(roots):
    """root_policy_temp 2 with eps 0.25 on 48 expanded roots of seeded priors and
    Dirichlet noise, GPU against the oracle.  The tempered path goes through powf:
    the host's is correctly rounded, the device's is accurate to about 1 ulp, so a
    tempered term may differ in the last place; the renormalising sum over up to
    ~100 children adds those differences up and the quotient carries both.  Priors
    agree within 8 float32 ulp (measured: about 28% of the 3,625 priors differ, by
    at most 4 ulp); every other tree array bit for bit.  The closed-form known
    answers (test_root_noise_known_answers, exact roots) hold to 2 ulp on both."""
    B = roots.shape[0]
    res = {}
    for name, eng in (("gpu", GpuEngine()), ("oracle", OracleEngine())):
        r = np.random.default_rng(11)
        t = eng.tree(B, 4096)
        legal, n = eng.legal(roots)
        pri, _, cq = synthetic_eval(r, n, B)
        results = roots[:, 3415].astype(np.int32)
        leaf0 = np.where((results == 0) & (n > 0), 0, -1).astype(np.int32)
        eng.expand_dense(t, cq, leaf0, roots, legal, n, pri, results)
        pad = int(np.maximum(n, 1).max())
        noise = np.zeros((B, pad), np.float32)
        for i in range(B):
            noise[i, : n[i]] = r.dirichlet([0.3] * max(1, n[i]))[: n[i]]
        eng.root_noise(t, noise, 0.25, 2.0)
        res[name] = eng.to_np(t)
    g, o = res["gpu"], res["oracle"]
    assert tree_equal(o, g) in ([], ["prior"])
    ulps = np.abs(g["prior"].astype(np.float64) - o["prior"]) / np.spacing(np.abs(o["prior"])).astype(np.float64)
    print(f"root noise at T=2: {int((ulps > 0).sum())} of {int(o['num_children'][:, 0].sum())} priors differ, "
          f"max {ulps.max():.2f} ulp")
    assert ulps.max() <= 8.0
    assert (o["prior"][:, 0] == 0).all()  # the roots' own priors are never touched


@pytest.mark.parametrize("mode", ["slots", "mask"])
def test_q_penalty_known_answers(oracle, mode):
    """The hand-worked q_penalty case (tests/mcts_driver.py) through the GPU selects and
    expansion + backup: same choices, visit counts, values and penalties as worked out."""
    from mcts_driver import check_q_penalty_case
    check_q_penalty_case(GpuEngine(), oracle.init_state(0), mode)


def test_expand_backprop_paths_not_chains(roots):
    """Virtual-loss paths that end at the leaf but are not selection chains (a middle
    entry swapped for a node of another subtree) take the reference's serial walk --
    the virtual-loss undo over the listed entries, the backup up the leaf's parents --
    in both GPU entry points: identical to the oracle, and the planned entry leaves
    those games to the one-wave order (no two waves write one subtree)."""
    import torch
    oe = OracleEngine()
    t, _ = run_search(oe, roots, W=2, C=4, M=8192, waves=5)
    B = roots.shape[0]
    slots = np.tile(np.arange(4, dtype=np.int32), (B, 1))
    slots[t["num_children"][:, 0][:, None] <= np.arange(4)[None, :]] = -1
    active = (t["num_children"][:, 0] > 0).astype(np.int8)
    leaf, paths, plen, vl, vlen = oe.select_slots(t, active, slots, 256, 1.25, 2)
    deep = np.nonzero(vlen >= 3)[0]
    assert len(deep) >= 8
    rng = np.random.default_rng(9)
    for s in deep[::2]:  # every other deep path: its second entry becomes another node of the game
        g = s % B
        other = int(rng.integers(1, t["node_count"][g]))
        while other in vl[s, : vlen[s]]:
            other = int(rng.integers(1, t["node_count"][g]))
        vl[s, 1] = other
    leaves = oe.replay(roots, paths, plen, leaf)
    lm, ln = oe.legal(leaves)
    p2, v2, q2 = synthetic_eval(rng, ln, leaf.shape[0])
    res = leaves[:, 3415].astype(np.int32)
    outs = []
    for eng in (GpuEngine(), _OneWavePerGame()):
        gt = {k: eng.c(v.copy()) for k, v in t.items()}
        eng.expand_backprop(gt, q2, leaf, leaves, lm, ln, p2, res, v2, vl, vlen)
        torch.cuda.synchronize()
        outs.append(eng.to_np(gt))
    oe.expand_backprop(t, q2, leaf, leaves, lm, ln, p2, res, v2, vl, vlen)
    assert tree_equal(t, outs[0]) == []
    assert tree_equal(t, outs[1]) == []
