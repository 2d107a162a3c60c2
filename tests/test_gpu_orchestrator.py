"""Gumbel self-play orchestrator on the GPU, every tree call shadowed by the oracle.

A real search ply (FNN `large`, seeded) runs through
hive_neuralnet_amd.orchestrator; each MCTS entry point it calls
(root expansion, root noise, root-slot selection, replay, expansion + backup)
is wrapped so that the same call, with the same inputs copied to the host, is
applied to a host mirror of the tree by the C tree oracle.  Outputs and the
whole tree must stay bit-identical after every call.  The network itself runs
in torch fp32 on the GPU; its outputs are inputs of the shadowed calls, so the
check covers the orchestrator's tree traffic exactly.
"""
import numpy as np
import pytest

from mcts_driver import record_wave_evaluations, tree_equal

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().numpy()


class Shadow:
    """Mirror of one orchestrator tree on the host, advanced by the oracle."""

    def __init__(self, orch, tree, monkeypatch):
        from oracle.mcts import MctsOracle
        orch.use_graphs = False  # every call is checked on the host as it happens
        self.m = MctsOracle()
        self.orch, self.tree = orch, tree
        self.calls = {}
        self.sync()
        ext = orch.ext
        for name in ("mcts_expand_dense_priors_batch", "mcts_apply_root_noise", "mcts_select_with_root_slots_batch",
                     "mcts_select_with_root_mask_batch", "mcts_replay_batch", "mcts_replay_fill_batch",
                     "mcts_expand_and_backprop_dense_priors_batch"):
            monkeypatch.setattr(ext, name, self._wrap(name, getattr(ext, name)), raising=False)
        # native waves (one library call each): the same select, replay and
        # expansion + backup applied to the mirror from the wave's buffers
        from hive_neuralnet_amd import hive_gpu
        real_run = hive_gpu.WavePlan.run

        def run(plan, *a, **k):
            out = real_run(plan, *a, **k)
            self._wave_run(plan, a)
            for name in ("mcts_select_with_root_slots_batch", "mcts_replay_fill_batch",
                         "mcts_expand_and_backprop_dense_priors_batch"):
                self.calls[name] = self.calls.get(name, 0) + 1
            self.check_tree("native wave")
            return out
        monkeypatch.setattr(hive_gpu.WavePlan, "run", run)

    def sync(self):
        self.ot = {k: _np(v).copy() for k, v in self.tree.items()}

    def check_tree(self, where):
        gt = {k: _np(v) for k, v in self.tree.items()}
        bad = tree_equal(self.ot, gt)
        assert bad == [], f"{where}: tree arrays differ: {bad}"

    def _wrap(self, name, fn):
        def call(*a):
            out = fn(*a)
            getattr(self, "_" + name)(a, out)
            self.calls[name] = self.calls.get(name, 0) + 1
            self.check_tree(name)
            return out
        return call

    def _mcts_expand_dense_priors_batch(self, a, out):
        cq, leaf, st, lm, nl, pri, res = [_np(x) for x in a[13:20]]
        was = self.m.expand_dense(self.ot, cq, leaf, st, lm, nl, pri, res)
        assert np.array_equal(was, _np(out))

    def _mcts_apply_root_noise(self, a, out):
        noise, roots = _np(a[12]), _np(a[13])
        self.m.root_noise(self.ot, noise, roots, float(a[15]), float(a[16]))

    def _mcts_select_with_root_slots_batch(self, a, out):
        active, roots, slots = _np(a[13]), _np(a[14]), _np(a[15])
        max_root, c_puct, W = int(a[17]), float(a[18]), int(a[20])
        rest = list(a[22:]) + [False, 4.0, 0.0][len(a) - 22:]
        exp = self.m.select_slots(self.ot, active, roots, slots, max_root, c_puct, W, bool(rest[0]),
                                  float(rest[1]), float(rest[2]))
        for e, g in zip(exp, out):
            assert np.array_equal(e, _np(g))

    def _mcts_select_with_root_mask_batch(self, a, out):
        active, roots, alive = _np(a[13]), _np(a[14]), _np(a[15])
        c_puct, W = float(a[17]), int(a[19])
        rest = list(a[21:]) + [False, 4.0, 0.0][len(a) - 21:]
        exp = self.m.select_mask(self.ot, active, roots, alive, c_puct, W, bool(rest[0]), float(rest[1]),
                                 float(rest[2]))
        for e, g in zip(exp, out):
            assert np.array_equal(e, _np(g))

    def _mcts_replay_batch(self, a, out):
        roots, leaves, paths, plen, leaf = [_np(x) for x in a[:5]]
        exp = np.zeros_like(leaves)
        self.m.replay(roots, exp, paths, plen, leaf)
        assert np.array_equal(exp, leaves)

    def _mcts_replay_fill_batch(self, a, out):  # the buffer started uninitialised: idle rows must be zero
        self._mcts_replay_batch(a, out)

    def _mcts_expand_and_backprop_dense_priors_batch(self, a, out):
        cq, leaf, st, lm, nl, pri, res, vals, vl, vlen = [_np(x) for x in a[13:23]]
        self.m.expand_backprop_dense(self.ot, cq, leaf, st, lm, nl, pri, res, vals, vl, vlen, float(a[26]))

    def _wave_run(self, plan, a):
        roots, active, rnodes, slots = [_np(x) for x in a[:4]]
        C, max_root, c_puct, W = int(a[4]), int(a[5]), float(a[6]), int(a[7])
        det, sigma, qp = bool(a[8]), float(a[9]), float(a[10])
        T = W * C * plan.B
        b = {k: _np(getattr(plan, k)[:T]) for k in (
            "leaf_idx", "move_paths", "path_lens", "vl_paths", "vl_lens", "leaf_states", "results", "legal_moves",
            "num_legal", "priors", "values", "child_q")}
        exp = dict(zip(("leaf_idx", "move_paths", "path_lens", "vl_paths", "vl_lens"),
                       self.m.select_slots(self.ot, active, rnodes, slots, max_root, c_puct, W, det, sigma, qp)))
        for k in ("leaf_idx", "path_lens", "vl_lens"):
            assert np.array_equal(exp[k], b[k]), f"native wave: select output {k} differs"
        # the wave writes each path row up to its recorded length (its readers stop there)
        depth = np.arange(exp["vl_paths"].shape[1])[None, :]
        rec = depth < b["path_lens"][:, None]
        assert np.array_equal(exp["move_paths"][rec], b["move_paths"][rec]), "native wave: move paths differ"
        rec = depth < b["vl_lens"][:, None]
        assert np.array_equal(exp["vl_paths"][rec], b["vl_paths"][rec]), "native wave: node paths differ"
        leaves = np.zeros_like(b["leaf_states"])
        self.m.replay(roots, leaves, b["move_paths"], b["path_lens"], b["leaf_idx"])
        assert np.array_equal(leaves, b["leaf_states"]), "native wave: replayed leaf states differ"
        assert np.array_equal(leaves[:, 3415].astype(np.int32), b["results"]), "native wave: leaf results differ"
        self.m.expand_backprop_dense(self.ot, b["child_q"], b["leaf_idx"], leaves, b["legal_moves"], b["num_legal"],
                                     b["priors"], b["results"], b["values"], b["vl_paths"], b["vl_lens"], qp)


def _setup(B, sims, M, mask, max_ply, seed, **kw):
    import torch
    from hive_neuralnet_amd import hive_gpu
    from hive_neuralnet_amd.fnn import seeded_large
    from hive_neuralnet_amd.orchestrator import FNNMCTSConfig, FNNMCTSOrchestrator
    net = seeded_large(seed)
    cfg = FNNMCTSConfig(num_simulations=sims, batch_size=B, max_tree_nodes=M, **kw)
    orch = FNNMCTSOrchestrator(net, cfg)
    states, _ = hive_gpu.random_positions(B, mask, max_ply, seed)
    torch.manual_seed(seed + 1)
    np.random.seed(seed)
    return orch, states, orch._alloc_tree(B)


@pytest.mark.parametrize("sims,M,mask,max_ply,kw", [
    (64, 4096, 7, 40, {}),
    (64, 600, 0, 30, {}),                       # node pool runs out mid-search
    (32, 4096, 7, 60, {"wave_parallel": False}),
], ids=["schedule", "pool-exhaustion", "w1"])
def test_search_ply_tree_calls_match_oracle(monkeypatch, sims, M, mask, max_ply, kw):
    import torch
    B = 12
    orch, states, tree = _setup(B, sims, M, mask, max_ply, 11, **kw)
    sh = Shadow(orch, tree, monkeypatch)
    active = torch.ones((B,), dtype=torch.bool, device="cuda")
    r = orch.search_ply(states, tree, active)
    assert sh.calls.get("mcts_expand_and_backprop_dense_priors_batch", 0) > 0
    assert sh.calls.get("mcts_replay_fill_batch", 0) == sh.calls["mcts_select_with_root_slots_batch"]
    sh.check_tree("end of ply")
    # the chosen slot is a legal move and the policy is a distribution over legal slots
    n = _np(r.num_legal)
    has = _np(r.has_actions)
    ch = _np(r.chosen_slot)
    pol = _np(r.policy)
    assert (ch[has] < n[has]).all()
    for i in np.nonzero(has)[0]:
        assert abs(pol[i].sum() - 1.0) < 1e-5
        assert (pol[i, n[i]:] == 0).all()
    # root visits = completed simulations through the root (pool exhaustion backs up too)
    vc = _np(tree["visit_count"])
    fc = _np(tree["first_child"])
    sv = _np(r.slot_visits)
    searched = has & (fc[:, 0] >= 0)
    assert searched.any()
    for i in np.nonzero(searched)[0]:
        assert vc[i, 0] == sv[i].sum() > 0


def test_two_plies_rebase_and_continue(monkeypatch):
    import torch
    B = 8
    orch, states, tree = _setup(B, 32, 4096, 0, 20, 5)
    sh = Shadow(orch, tree, monkeypatch)
    active = torch.ones((B,), dtype=torch.bool, device="cuda")
    for ply in range(2):
        r = orch.search_ply(states, tree, active)
        sh.check_tree(f"ply {ply}")
        before = states.clone()
        orch.apply_and_rebase(states, tree, r)
        moved = _np(r.has_actions)
        assert (_np(tree["node_count"])[moved] == 1).all()
        assert (_np(tree["first_child"])[moved] == -1).all()
        assert not torch.equal(before[torch.from_numpy(moved).cuda()], states[torch.from_numpy(moved).cuda()])
        sh.sync()


def test_self_play_batch_examples():
    import torch
    from hive_neuralnet_amd.fnn import seeded_large
    from hive_neuralnet_amd.orchestrator import FNNMCTSConfig, FNNMCTSOrchestrator
    net = seeded_large(3)
    cfg = FNNMCTSConfig(num_simulations=16, batch_size=4, max_tree_nodes=2048, max_game_length=6)
    torch.manual_seed(4)
    np.random.seed(4)
    ex = FNNMCTSOrchestrator(net, cfg).self_play_batch()
    assert len(ex) == 4
    for game in ex:
        assert 1 <= len(game) <= 6
        for e in game:
            assert e.state_bytes.shape == (3424,) and e.state_bytes.dtype == np.uint8
            assert abs(float(e.policy_target.sum()) - 1.0) < 1e-5
            assert e.value_target in (-1.0, 0.0, 1.0)


@pytest.mark.parametrize("sims,mask,max_ply,seed,kw", [
    (64, 7, 40, 21, {}),
    (48, 0, 80, 22, {}),
    (32, 7, 60, 23, {"wave_parallel": False}),
], ids=["mask7", "mask0-late", "w1"])
def test_search_ply_matches_numpy_orchestrator(monkeypatch, sims, mask, max_ply, seed, kw):
    """The torch orchestrator's host logic against oracle/orchestrator.py (numpy),
    fed the same recorded network outputs, Gumbel draws and Dirichlet noise.

    The seeded cases cover queen-surround reserve slots (6-8 games per case),
    a finished game (mask0-late), and an immediate win, which also clears
    every other game's priors (w1)."""
    import torch
    from oracle.orchestrator import SearchPlyOracle
    B = 12
    orch, states, tree = _setup(B, sims, 1 << 15, mask, max_ply, seed, **kw)
    evals, uniforms, noises = [], [], []
    real_eval = orch._eval_states

    def rec_eval(*a, **k):
        out = real_eval(*a, **k)
        evals.append(tuple(_np(x).copy() for x in out))
        return out

    real_rand = torch.rand

    def rec_rand(*a, **k):
        out = real_rand(*a, **k)
        uniforms.append(_np(out).copy())
        return out

    ext = orch.ext
    real_noise = ext.mcts_apply_root_noise

    def rec_noise(*a):
        noises.append(_np(a[12]).copy())
        return real_noise(*a)

    monkeypatch.setattr(orch, "_eval_states", rec_eval)
    monkeypatch.setattr(torch, "rand", rec_rand)
    monkeypatch.setattr(ext, "mcts_apply_root_noise", rec_noise, raising=False)
    record_wave_evaluations(monkeypatch, evals)
    orch.use_graphs = False  # the recording reads every evaluation on the host
    t0 = {k: _np(v).copy() for k, v in tree.items()}
    st = _np(states).copy()
    active = torch.ones((B,), dtype=torch.bool, device="cuda")
    r = orch.search_ply(states, tree, active)
    assert len(uniforms) == 1 and len(noises) == 1 and len(evals) >= 2

    ref = SearchPlyOracle(orch.config)
    legal, n, _, _ = ref.o.batch_legal_features_actions(st, want_features=False, want_actions=False)
    assert np.array_equal(legal, _np(r.legal_moves)) and np.array_equal(n, _np(r.num_legal))
    chosen, probs, visits = ref.run(t0, st, np.ones(B, bool), legal, n, evals[0], uniforms[0], noises[0], evals[1:])
    assert np.array_equal(chosen, _np(r.chosen_slot))
    assert np.array_equal(visits, _np(r.slot_visits))
    np.testing.assert_allclose(probs, _np(r.policy), atol=2e-6, rtol=0)
    assert tree_equal(t0, {k: _np(v) for k, v in tree.items()}) == []


@pytest.mark.parametrize("seed,mask,max_ply", [(31, 0, 120), (32, 7, 150)])
def test_fused_leaf_evaluation_matches_torch(seed, mask, max_ply):
    """hg_fnn_leaf_eval (network and heads on fp32 matrix cores) against the
    reference's torch composition over HiveFNN (fnn_network.py:175-220,
    fnn_mcts_orchestrator.py:243-316) and against the network restated in
    float64 numpy, on 2,000 leaves and every legal successor.

    Priors: within 1e-5 relative of float64, with no absolute floor (both
    paths measure ~3e-7).  Values and child Q are tanh outputs of 64-term fp32
    dot products: both paths carry ~5e-7 absolute error, so near 0 no fp32
    path meets a bare relative bound (torch's own fp32 composition is 2-4e-5
    relative off float64 even above 0.01).  The bar there is torch's own
    measured floor: fused within rtol 1e-5 + floor of torch, floor = torch's
    largest absolute error against float64 in this same test (so the fused
    path is within rtol 1e-5 + 2 floor of float64)."""
    import torch
    from hive_neuralnet_amd import hive_gpu
    B = 2000
    orch, _, _ = _setup(4, 8, 256, mask, max_ply, seed)
    ext = orch.ext
    states, _ = hive_gpu.random_positions(B, mask, max_ply, 77 + seed)
    legal, nl, feat = ext.generate_legal_moves_and_fnn_features_batch(states, B)
    orch._head_biases = (float(orch.net.value_fc.bias.item()), float(orch.net.action_fc2.bias.item()))
    p1, v1, q1 = orch._eval_states(states, legal, nl, B, feat)
    p2, v2, q2 = orch._eval_states_torch(states, legal, nl, B, feat)
    n = nl.cpu().numpy()
    pr = p1.cpu().numpy()
    assert (pr[np.arange(256)[None, :] >= n[:, None]] == 0).all()
    live = n > 0
    np.testing.assert_allclose(pr[live].sum(axis=1), 1.0, atol=1e-5)

    # the network restated in float64 over the same features
    a2r = np.repeat(np.arange(B), n).astype(np.int64)
    mi = np.concatenate([np.arange(k) for k in n]).astype(np.int64)
    succ = ext.fnn_successor_features_batch(states, legal, torch.from_numpy(a2r).cuda(), torch.from_numpy(mi).cuda(),
                                            len(a2r))
    W = {k: v.detach().double().cpu().numpy() for k, v in orch.net.state_dict().items()}

    def enc(x):
        h = 1 / (1 + np.exp(-(x @ W["fc1.weight"].T + W["fc1.bias"])))
        h = (h - h.mean(1, keepdims=True)) / np.sqrt(h.var(1, keepdims=True) + 1e-5)
        return (h * W["ln1.weight"] + W["ln1.bias"]) @ W["fc2.weight"].T + W["fc2.bias"]

    er, es = enc(_np(feat).astype(np.float64)), enc(_np(succ).astype(np.float64))
    val = lambda e: np.tanh(e @ W["value_fc.weight"].T + W["value_fc.bias"])[:, 0]  # noqa: E731
    z = 1 / (1 + np.exp(-(np.concatenate([er[a2r], es], 1) @ W["action_fc1.weight"].T + W["action_fc1.bias"])))
    logit = (z @ W["action_fc2.weight"].T + W["action_fc2.bias"])[:, 0]
    want_p = np.zeros((B, 256))
    want_q = np.zeros((B, 256))
    cv = -val(es)
    offs = np.concatenate([[0], np.cumsum(n)])
    for t in range(B):
        s = slice(int(offs[t]), int(offs[t + 1]))
        if n[t] > 0:
            x = np.exp(logit[s] - logit[s].max())
            want_p[t, :n[t]] = x / x.sum()
            want_q[t, :n[t]] = cv[s]
    slots = np.arange(256)[None, :] < n[:, None]
    # priors: 1e-5 relative of float64, no floor, both paths; fused vs torch likewise
    np.testing.assert_allclose(pr[slots], want_p[slots], rtol=1e-5, atol=0)
    np.testing.assert_allclose(_np(p2)[slots], want_p[slots], rtol=1e-5, atol=0)
    np.testing.assert_allclose(pr[slots], _np(p2)[slots], rtol=1e-5, atol=0)
    for fused, ref, want in ((_np(v1), _np(v2), val(er)), (_np(q1)[slots], _np(q2)[slots], want_q[slots])):
        floor = float(np.abs(ref.astype(np.float64) - want).max())  # torch fp32's own error
        assert floor < 1e-6
        np.testing.assert_allclose(fused, ref, rtol=1e-5, atol=floor)
        np.testing.assert_allclose(fused, want, rtol=1e-5, atol=2 * floor)


@pytest.mark.parametrize("M", [4096, 600], ids=["roomy", "pool-exhausted"])
def test_reset_trees_equals_full_refill(M):
    """hg_mcts_reset_trees (used prefix only) against the reference's hard
    rebase, which refills every node of the reset games' rows
    (fnn_mcts_orchestrator.py:1122-1142), on trees left by a real search ply."""
    import torch
    B = 8
    orch, states, tree = _setup(B, 64, M, 7, 40, 13)
    active = torch.ones((B,), dtype=torch.bool, device="cuda")
    orch.search_ply(states, tree, active)
    cnt = _np(tree["node_count"])
    assert (cnt > 1).all() and cnt.max() <= M
    reset = torch.tensor([1, 0, 1, 1, 0, 1, 0, 1], dtype=torch.bool, device="cuda")
    rows = torch.nonzero(reset).squeeze(1)
    expect = {k: v.clone() for k, v in tree.items()}
    for k, fill in (("visit_count", 0), ("total_value", 0), ("prior", 0), ("parent_idx", -1), ("move_bytes", 0),
                    ("action_idx", -1), ("first_child", -1), ("num_children", 0), ("is_terminal", 0),
                    ("terminal_value", 0), ("child_init_q", 0)):
        expect[k][rows] = fill
    expect["node_count"][rows] = 1
    expect["root_node"][rows] = 0
    orch._reset_games(tree, reset)
    assert tree_equal({k: _np(v) for k, v in expect.items()}, {k: _np(v) for k, v in tree.items()}) == []


@pytest.mark.parametrize("mask,max_ply,wave_parallel,mode", [(0, 60, True, "waves"), (7, 90, True, "waves"),
                                                             (0, 40, False, "waves"), (0, 60, True, "ply"),
                                                             (7, 90, False, "ply"), (0, 60, True, "ply2"),
                                                             (7, 90, False, "ply3")])
def test_graph_waves_equal_eager(mask, max_ply, wave_parallel, mode):
    """Simulation waves replayed from captured HIP graphs -- one graph per wave
    shape ("waves"), or the whole search phase of a ply, every wave of the four
    rounds and the halving decisions, as one graph ("ply"; "ply2" / "ply3":
    the games in two / three ranges whose waves are parallel branches of the
    graph) -- against the same waves run eagerly: three plies (so each graph
    is replayed across rounds, plies and tree rebases, with eager work and
    host reads in between), every ply's choice, policy and visits, the search
    counters and the final trees bit-identical."""
    import torch
    from hive_neuralnet_amd import hive_gpu
    outs = []
    for graphs in (False, True):
        B = 16
        orch, _, tree = _setup(B, 64, 8192, mask, max_ply, 71, wave_parallel=wave_parallel)
        if not graphs:
            orch.use_graphs, orch.use_ply_graphs = False, False
        elif mode == "waves":
            orch.use_graphs, orch.use_ply_graphs = True, False
        else:
            orch.use_graphs, orch.use_ply_graphs = None, True
            orch.ply_graph_parts = {"ply": 1, "ply2": 2, "ply3": 3}[mode]
        orch.enable_counters()
        states, _ = hive_gpu.random_positions(B, mask, max_ply, 72)
        torch.manual_seed(73)
        np.random.seed(73)
        active = torch.ones((B,), dtype=torch.bool, device="cuda")
        rec = []
        for _ in range(3):
            r = orch.search_ply(states, tree, active)
            rec.append((_np(r.chosen_slot), _np(r.policy), _np(r.slot_visits)))
            orch.apply_and_rebase(states, tree, r)
            active &= orch.ext.check_results_batch(states, B) == 0
        rec.append(_np(orch._stats).copy())
        rec.append({k: _np(v).copy() for k, v in tree.items()})
        if graphs:
            assert len(orch._graphs if mode == "waves" else orch._ply_graphs) >= 1
        else:
            assert not orch._graphs and not orch._ply_graphs
        outs.append(rec)
    for a, b in zip(outs[0][:-2], outs[1][:-2]):
        for x, y in zip(a, b):
            assert np.array_equal(x.view(np.uint32) if x.dtype == np.float32 else x,
                                  y.view(np.uint32) if y.dtype == np.float32 else y)
    assert np.array_equal(outs[0][-2], outs[1][-2])
    assert tree_equal(outs[0][-1], outs[1][-1]) == []


def test_root_dirichlet_noise_rows(monkeypatch):
    """_apply_root_dirichlet: one Dirichlet draw per active game over its root
    children (rows sum to 1 on exactly the first num_children entries),
    nothing for idle games; the mean over games of each row's first entry
    is 1/n, as Dirichlet(alpha, ..., alpha) gives."""
    import torch
    B = 64
    orch, states, tree = _setup(B, 16, 4096, 0, 30, 5)
    ext = orch.ext
    legal, nl, feat = ext.generate_legal_moves_and_fnn_features_batch(states, B)
    orch._head_biases = (float(orch.net.value_fc.bias.item()), float(orch.net.action_fc2.bias.item()))
    priors, _, cq = orch._eval_states(states, legal, nl, B, feat)
    act = torch.ones((B,), dtype=torch.bool, device="cuda")
    act[::5] = False
    orch._expand_root_if_needed(tree, states, legal, nl, priors, cq, act.to(torch.int8), B)
    got = []
    monkeypatch.setattr(ext, "mcts_apply_root_noise", lambda *a: got.append(_np(a[12]).copy()), raising=False)
    np.random.seed(3)
    draws = []
    for _ in range(200):
        orch._apply_root_dirichlet(tree, B, act)
        draws.append(got[-1])
    nc = _np(tree["num_children"][torch.arange(B, device="cuda"), tree["root_node"]])
    a = _np(act)
    for d in draws:
        for i in range(B):
            n = int(nc[i])
            if not a[i] or n == 0:
                assert not d[i].any()
            else:
                assert abs(float(d[i, :n].sum()) - 1.0) < 1e-5 and not d[i, n:].any() and (d[i, :n] >= 0).all()
    first = np.array([d[:, 0] for d in draws])  # [draws, B]
    for i in np.nonzero(a & (nc > 1))[0]:
        assert abs(first[:, i].mean() - 1.0 / nc[i]) < 0.12


@pytest.mark.parametrize("mask,max_ply,parts", [(0, 60, 2), (7, 90, 3)])
def test_game_ranges_on_streams_equal_one_range(mask, max_ply, parts):
    """Simulation waves of disjoint game ranges on their own streams
    (game_parts) against one range on the current stream: three plies with
    rebases, every ply's choice, policy and visits, the wave counters and the
    final trees identical."""
    import torch
    from hive_neuralnet_amd import hive_gpu
    outs = []
    for gp in (1, parts):
        B = 18
        orch, _, tree = _setup(B, 64, 8192, mask, max_ply, 81)
        orch.game_parts = gp
        orch.use_graphs = False
        orch.enable_counters()
        states, _ = hive_gpu.random_positions(B, mask, max_ply, 82)
        torch.manual_seed(83)
        np.random.seed(83)
        active = torch.ones((B,), dtype=torch.bool, device="cuda")
        rec = []
        for _ in range(3):
            r = orch.search_ply(states, tree, active)
            rec.append((_np(r.chosen_slot), _np(r.policy), _np(r.slot_visits)))
            orch.apply_and_rebase(states, tree, r)
            active &= orch.ext.check_results_batch(states, B) == 0
        rec.append(_np(orch._stats).copy())
        rec.append({k: _np(v).copy() for k, v in tree.items()})
        outs.append(rec)
    for a, b in zip(outs[0][:3], outs[1][:3]):
        for x, y in zip(a, b):
            assert np.array_equal(x.view(np.uint32) if x.dtype == np.float32 else x,
                                  y.view(np.uint32) if y.dtype == np.float32 else y)
    assert np.array_equal(outs[0][3], outs[1][3])
    assert tree_equal(outs[0][4], outs[1][4]) == []


@pytest.mark.parametrize("mask,max_ply,M,parts,kw", [
    (0, 60, 8192, 1, {}),
    (7, 90, 8192, 1, {"wave_parallel": False}),
    (7, 90, 8192, 2, {}),
    (0, 30, 600, 1, {}),                        # node pool runs out mid-search
], ids=["schedule", "w1", "two-ranges", "pool-exhaustion"])
def test_native_waves_equal_step_waves(mask, max_ply, M, parts, kw):
    """Simulation waves as one library call (hg_mcts_wave_root_slots through
    WavePlan) against the same waves through the step entry points (select,
    replay, results, legal + features, leaf evaluation, expansion + backup):
    three plies with rebases, every ply's choice, policy and visits, the wave
    counters and the final trees bit-identical."""
    import torch
    from hive_neuralnet_amd import hive_gpu
    outs = []
    for native in (False, True):
        B = 18
        orch, _, tree = _setup(B, 64, M, mask, max_ply, 91, **kw)
        orch.native_waves = native
        orch.game_parts = parts
        orch.use_graphs = False
        orch.enable_counters()
        states, _ = hive_gpu.random_positions(B, mask, max_ply, 92)
        torch.manual_seed(93)
        np.random.seed(93)
        active = torch.ones((B,), dtype=torch.bool, device="cuda")
        rec = []
        for _ in range(3):
            r = orch.search_ply(states, tree, active)
            rec.append((_np(r.chosen_slot), _np(r.policy), _np(r.slot_visits)))
            orch.apply_and_rebase(states, tree, r)
            active &= orch.ext.check_results_batch(states, B) == 0
        assert bool(orch._wave_plans) == native
        rec.append(_np(orch._stats).copy())
        rec.append({k: _np(v).copy() for k, v in tree.items()})
        outs.append(rec)
    for a, b in zip(outs[0][:3], outs[1][:3]):
        for x, y in zip(a, b):
            assert np.array_equal(x.view(np.uint32) if x.dtype == np.float32 else x,
                                  y.view(np.uint32) if y.dtype == np.float32 else y)
    assert np.array_equal(outs[0][3], outs[1][3])
    assert tree_equal(outs[0][4], outs[1][4]) == []


def test_wave_plan_rejects_oversized_wave():
    """A wave of more simulations than the plan's buffers hold is refused
    before any launch; a smaller one runs."""
    import torch
    B = 4
    orch, states, tree = _setup(B, 16, 2048, 0, 20, 7)
    orch._head_biases = (float(orch.net.value_fc.bias.item()), float(orch.net.action_fc2.bias.item()))
    plan = orch.ext.prepare_wave_root_slots(*orch._tree_args(tree), tree["child_init_q"], B, 2048, orch.net,
                                            orch._head_biases, capacity=2 * B)
    active = torch.zeros((B,), dtype=torch.int8, device="cuda")
    slots = torch.full((B, 2), -1, dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError, match="capacity"):
        plan.run(states, active, tree["root_node"], slots, 2, 256, 1.25, 2)
    leaf, _, _, _ = plan.run(states, active, tree["root_node"], slots, 2, 256, 1.25, 1)
    assert (_np(leaf) == -1).all()  # no active game: every simulation idle


def _bare_orch(**over):
    from hive_neuralnet_amd.fnn import seeded_large
    from hive_neuralnet_amd.orchestrator import FNNMCTSConfig, FNNMCTSOrchestrator
    return FNNMCTSOrchestrator(seeded_large(1), FNNMCTSConfig(**over))


@pytest.mark.parametrize("name", ["k16-schedule", "k16-w1", "k64-schedule"])
def test_sequential_halving_known_answers(name):
    """FNNMCTSOrchestrator._sequential_halving against the hand-worked cases
    of tests/orchestrator_cases.py (the same ones the numpy restatement meets)."""
    import torch
    from orchestrator_cases import HALVING_CASES, HalvingStub, halving_base
    over, rows, calls, chosen = HALVING_CASES[name]
    orch = _bare_orch(**over)
    stub = HalvingStub()

    def stats(c):
        v, q = stub.child_stats(c.cpu().numpy())
        return torch.from_numpy(v).cuda(), torch.from_numpy(q).cuda()

    cand = torch.tensor(rows, dtype=torch.int32, device="cuda")
    got, sims = orch._sequential_halving(cand, torch.from_numpy(halving_base(len(rows))).cuda(),
                                         lambda c, ps, w: stub.run_round(c.cpu().numpy(), ps, w), stats)
    assert stub.calls == calls
    assert got.cpu().tolist() == chosen
    assert sims == sum(ps * len(r[0]) * len(r) for r, ps, _ in calls)


@pytest.mark.parametrize("name", ["k16-schedule", "k16-w1", "k64-schedule"])
def test_halving_kernel_known_answers(name):
    """The same hand-worked halving cases through hg_gumbel_halving: each
    round's statistics are written into a tree (root 0, its 256 children at
    nodes 1-256: N = the stub's visits, W = -Q * N), and every decision --
    survivors and the final choice -- is the kernel's."""
    import torch
    from orchestrator_cases import HALVING_CASES, HalvingStub, halving_base, q_of
    over, rows, calls, chosen = HALVING_CASES[name]
    orch = _bare_orch(**over)
    B = len(rows)
    tree = orch._alloc_tree(B)
    tree["first_child"][:, 0] = 1
    tree["num_children"][:, 0] = 256
    stub = HalvingStub()
    hg_tree = orch.ext.tree_struct(*orch._tree_args(tree), tree["child_init_q"], B, tree["visit_count"].shape[1])
    base = torch.from_numpy(halving_base(B)).cuda()

    def run_round(c, ps, w):
        n = stub.run_round(c.cpu().numpy(), ps, w)
        r = len(stub.calls) - 1
        vc = np.zeros((B, 256), np.int32)
        tv = np.zeros((B, 256), np.float32)
        for (g, slot), v in stub.visits.items():
            vc[g, slot] = v
            tv[g, slot] = np.float32(-np.float32(q_of(r, g, slot)) * np.float32(v))
        tree["visit_count"][:, 1:257] = torch.from_numpy(vc).cuda()
        tree["total_value"][:, 1:257] = torch.from_numpy(tv).cuda()
        return n

    def decide(c, final):
        return orch.ext.gumbel_halving(hg_tree, tree["root_node"], c.contiguous(), base, orch.config.c_visit,
                                       orch.config.c_scale, 0, final)

    cand = torch.tensor(rows, dtype=torch.int32, device="cuda")
    got, sims = orch._sequential_halving(cand, base, run_round, None, decide)
    assert stub.calls == calls
    assert got.cpu().tolist() == chosen


@pytest.mark.parametrize("k,kw", [
    (16, {}), (16, {"wave_parallel": False}), (5, {}), (64, {"root_q_min_visits": 3}), (3, {"c_scale": 0.1}),
], ids=["k16", "k16-w1", "k5", "k64-minvisits", "k3-scale"])
def test_native_halving_equals_torch(k, kw):
    """Sequential halving decided by hg_gumbel_halving against the torch ops
    on the same searches: three plies with rebases, every ply's choice,
    policy and visits and the final trees bit-identical."""
    import torch
    from hive_neuralnet_amd import hive_gpu
    outs = []
    for native in (False, True):
        B = 24
        orch, _, tree = _setup(B, 128, 1 << 14, 7, 70, 101, max_num_considered_actions=k, **kw)
        orch.native_halving = native
        orch.use_graphs = False
        states, _ = hive_gpu.random_positions(B, 7, 70, 102)
        torch.manual_seed(103)
        np.random.seed(103)
        active = torch.ones((B,), dtype=torch.bool, device="cuda")
        rec = []
        for _ in range(3):
            r = orch.search_ply(states, tree, active)
            rec.append((_np(r.chosen_slot), _np(r.policy), _np(r.slot_visits)))
            orch.apply_and_rebase(states, tree, r)
            active &= orch.ext.check_results_batch(states, B) == 0
        assert (orch._packed is not None) == native
        rec.append({kk: _np(v).copy() for kk, v in tree.items()})
        outs.append(rec)
    for a, b in zip(outs[0][:3], outs[1][:3]):
        for x, y in zip(a, b):
            assert np.array_equal(x.view(np.uint32) if x.dtype == np.float32 else x,
                                  y.view(np.uint32) if y.dtype == np.float32 else y)
    assert tree_equal(outs[0][3], outs[1][3]) == []


@pytest.mark.parametrize("case", [0, 1])
def test_reserve_candidates_known_answers(case):
    """The reserve rule on the hand-built positions of tests/orchestrator_cases.py:
    qualifying moves (queen surround + escape on the GPU) and the candidate row."""
    import torch
    from orchestrator_cases import RESERVE_CASES, priors_formula
    build, n, want = RESERVE_CASES[case]
    for immobile, (qual_slots, row) in want.items():
        orch = _bare_orch(queen_surround_reserve_immobile_only=immobile)
        st = torch.from_numpy(build()[None]).cuda()
        legal, nl = orch.ext.generate_legal_moves_batch(st, 1)
        assert int(nl[0]) == n
        qual = orch._queen_surround_qualifying_mask(st, legal, nl, 1)
        assert torch.nonzero(qual[0]).squeeze(1).tolist() == qual_slots
        valid = orch._slot_idx < nl.to(torch.int64).unsqueeze(1)
        pri = torch.from_numpy(priors_formula(n)[None]).cuda()
        assert orch._candidate_row(qual, valid, pri, 16, 6)[0].tolist() == row


def test_candidate_row_short_list():
    import torch
    from orchestrator_cases import CANDIDATE_SHORT as c
    orch = _bare_orch()
    pri = torch.zeros((1, 256), dtype=torch.float32, device="cuda")
    pri[0, :c["n"]] = torch.tensor(c["priors"])
    qual = torch.zeros((1, 256), dtype=torch.bool, device="cuda")
    qual[0, c["qual"]] = True
    valid = orch._slot_idx < c["n"]
    assert orch._candidate_row(qual, valid, pri, 16, 6)[0].tolist() == c["row"]


@pytest.mark.parametrize("mask,max_ply,immobile", [(0, 120, True), (7, 150, True), (7, 150, False)])
def test_reserve_candidates_match_oracle(mask, max_ply, immobile):
    """hg_reserve_candidates (qualification + candidate row in one launch)
    against the numpy restatement (oracle/orchestrator.py: qualifying moves
    by the C oracle's apply and queen escape, candidate_row) on 768 seeded
    positions, the half whose opponent queen already has three or more
    occupied neighbours first (where moves qualify); with and without an
    allowed mask, and the candidate row from given masks (hg_candidate_rows)."""
    import torch
    from hive_neuralnet_amd import hive_gpu
    from hive_neuralnet_amd.orchestrator import FNNMCTSConfig
    from oracle.orchestrator import SearchPlyOracle, _surround, _turn, candidate_row
    ext = hive_gpu.load_extension()
    st, _ = hive_gpu.random_positions(4096, mask, max_ply, 0x5EED + 21)
    stn = _np(st)
    surround = np.array([_surround(s, (_turn(s) + 1) & 1) for s in stn])
    pick = np.concatenate([np.nonzero(surround >= 3)[0][:384], np.nonzero(surround < 3)[0][:384]])
    st = st[torch.from_numpy(pick).cuda()].contiguous()
    B = st.shape[0]
    legal, nl = ext.generate_legal_moves_batch(st, B)
    rng = np.random.default_rng(5)
    pri = rng.random((B, 256)).astype(np.float32)
    pri[:, ::7] = pri[:, 3::7][:, : pri[:, ::7].shape[1]]  # ties between slots
    allowed = rng.random((B, 256)) < 0.8
    cfg = FNNMCTSConfig(queen_surround_reserve_immobile_only=immobile)
    orc = SearchPlyOracle(cfg)
    want_q = orc.qualifying(_np(st), _np(legal), _np(nl))
    assert want_q.any(axis=1).sum() >= 50
    n = _np(nl)
    for al in (None, allowed):
        valid = np.arange(256)[None, :] < n[:, None]
        if al is not None:
            valid &= al
        want_c = candidate_row(want_q, valid, pri, 16, 6)
        q, c = ext.reserve_candidates(st, legal, nl, B, immobile, priors=torch.from_numpy(pri).cuda(), k=16,
                                      reserve=6, allowed=None if al is None else torch.from_numpy(al).cuda())
        assert np.array_equal(_np(q), want_q)
        assert np.array_equal(_np(c), want_c)
        c2 = ext.candidate_rows(torch.from_numpy(want_q).cuda(), torch.from_numpy(valid).cuda(),
                                torch.from_numpy(pri).cuda(), 16, 6)
        assert np.array_equal(_np(c2), want_c)
