"""The Gumbel self-play ply at its benchmark configuration (C5): 512 games,
4,096 simulations per move, k = 16 considered root actions, FNN `large`
(seeded random init), max_tree_nodes = 1 + 4096 * 256
(fnn_mcts_orchestrator.py:561-755; mcts_tree.cuh:811-1187).

Two checks per ply:

* every game's used node prefix satisfies the tree invariants: node_count =
  1 + the children of expanded nodes; each non-root node lies in its parent's
  child range; the root's visits equal the simulations the halving schedule
  gives that game and the sum of its children's; an expanded non-root node
  ended between 1 and W simulations itself (W = the most simulations one wave
  sends into one root child's subtree); every visited non-terminal node is
  expanded; no
  virtual-loss remainder (virtual_q_penalty 0, |W| <= N); root children are
  the root's legal list in order, with the reference's action indices;
* a slice of games in each game range is shadowed call by call by the C
  tree oracle: root expansion, root noise, every root-slot select (paths,
  leaves, virtual-loss paths), the replayed leaf states, their legal lists
  and results (from the oracle's own engine), and every expansion + backup fed
  the GPU network's outputs for those rows; at the end of the ply the
  shadowed trees must equal the GPU's array by array.

The schedule (2, 4, 8, 16) runs on the default two game ranges (two streams);
one simulation per candidate per wave runs on one range.
"""
import os

import numpy as np
import pytest

from mcts_driver import tree_equal

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]

GAMES, SIMS, K = 512, 4096, 16
MAX_NODES = 1 + SIMS * 256
# six games at the start of each game range, and two games (41, 488 from these
# seeded roots) whose candidate rows hold a reserve slot twice
SHADOW = list(range(0, 6)) + [41] + list(range(256, 262)) + [488]


def _np(t):
    return t.detach().cpu().numpy()


class SliceShadow:
    """Host mirror of the SHADOW games' trees, advanced by the C tree oracle
    on exactly the rows of those games in every tree call."""

    def __init__(self, orch, tree, monkeypatch, games=SHADOW):
        import torch
        from oracle.mcts import MctsOracle
        self.torch = torch
        self.m = MctsOracle()
        self.tree, self.games = tree, list(games)
        self.M = tree["visit_count"].shape[1]
        self.base = tree["visit_count"].data_ptr()
        self.calls = {}
        self.sync()
        ext = orch.ext
        for name in ("mcts_expand_dense_priors_batch", "mcts_apply_root_noise", "mcts_select_with_root_slots_batch",
                     "mcts_replay_fill_batch", "mcts_expand_and_backprop_dense_priors_batch"):
            monkeypatch.setattr(ext, name, self._wrap(name, getattr(ext, name)), raising=False)
        # native waves (one library call each): the same three steps checked
        # from the wave's buffers
        from hive_neuralnet_amd import hive_gpu
        real_run = hive_gpu.WavePlan.run

        def run(plan, *a, **k):
            out = real_run(plan, *a, **k)
            self._wave_run(plan, a)
            for name in ("mcts_select_with_root_slots_batch", "mcts_replay_fill_batch",
                         "mcts_expand_and_backprop_dense_priors_batch"):
                self.calls[name] = self.calls.get(name, 0) + 1
            return out
        monkeypatch.setattr(hive_gpu.WavePlan, "run", run)

    def sync(self):
        idx = self.torch.tensor(self.games, device="cuda")
        self.ot = {k: _np(v[idx]).copy() for k, v in self.tree.items()}

    def check(self, where):
        idx = self.torch.tensor(self.games, device="cuda")
        bad = tree_equal(self.ot, {k: _np(v[idx]) for k, v in self.tree.items()})
        assert bad == [], f"{where}: shadowed trees differ: {bad}"

    # -- which rows of a call belong to shadowed games --------------------
    def _blocks(self, first_game, B):
        """Per run of consecutive shadowed games inside the call's games
        [first_game, first_game + B): (mirror rows j0:j1, the call's local
        game ids).  Games are independent, so each run is its own oracle call."""
        out = []
        for j, g in enumerate(self.games):
            if first_game <= g < first_game + B:
                if out and out[-1][1][-1] == g - first_game - 1 and out[-1][0][1] == j:
                    out[-1][0][1] = j + 1
                    out[-1][1].append(g - first_game)
                else:
                    out.append(([j, j + 1], [g - first_game]))
        return out

    def _tree_blocks(self, a, B):
        return self._blocks((a[0].data_ptr() - self.base) // (4 * self.M), B)

    def _rows(self, T, B, local):
        r = (np.arange(T // B)[:, None] * B + np.asarray(local)[None, :]).reshape(-1)
        return self.torch.from_numpy(r).cuda()

    def _sub(self, js):
        return {k: v[js[0]:js[1]] for k, v in self.ot.items()}

    def _wrap(self, name, fn):
        def call(*a):
            out = fn(*a)
            getattr(self, "_" + name)(a, out)
            self.calls[name] = self.calls.get(name, 0) + 1
            return out
        return call

    # -- shadowed calls ----------------------------------------------------
    def _mcts_expand_dense_priors_batch(self, a, out):
        B, T = int(a[20]), int(a[21])
        for js, local in self._tree_blocks(a, B):
            r = self._rows(T, B, local)
            cq, leaf, st, lm, nl, pri, res = [np.ascontiguousarray(_np(x[r])) for x in a[13:20]]
            was = self.m.expand_dense(self._sub(js), cq, leaf, st, lm, nl, pri, res)
            assert np.array_equal(was, _np(out[r]))

    def _mcts_apply_root_noise(self, a, out):
        B = int(a[17])
        for js, local in self._tree_blocks(a, B):
            g = self.torch.tensor(local, device="cuda")
            self.m.root_noise(self._sub(js), np.ascontiguousarray(_np(a[12][g])), _np(a[13][g]), float(a[15]),
                              float(a[16]))

    def _mcts_select_with_root_slots_batch(self, a, out):
        B, W = int(a[19]), int(a[20])
        rest = list(a[22:]) + [False, 4.0, 0.0][len(a) - 22:]
        for js, local in self._tree_blocks(a, B):
            g = self.torch.tensor(local, device="cuda")
            exp = self.m.select_slots(self._sub(js), _np(a[13][g]), _np(a[14][g]),
                                      np.ascontiguousarray(_np(a[15][g])), int(a[17]), float(a[18]), W,
                                      bool(rest[0]), float(rest[1]), float(rest[2]))
            r = self._rows(W * int(a[16]) * B, B, local)
            for e, o in zip(exp, out):
                assert np.array_equal(e, _np(o[r])), "select outputs differ"

    def _mcts_replay_fill_batch(self, a, out):
        roots, leaves, paths, plen, leaf = a[:5]
        B, T = int(a[5]), int(a[6])
        # the replay takes root states, not tree views: the call's games by address
        for js, local in self._blocks((roots.data_ptr() - self.root_base) // 3424, B):
            r = self._rows(T, B, local)
            g = self.torch.tensor(local, device="cuda")
            exp = np.zeros((len(r), 3424), np.uint8)
            self.m.replay(np.ascontiguousarray(_np(roots[g])), exp, np.ascontiguousarray(_np(paths[r])),
                          np.ascontiguousarray(_np(plen[r])), np.ascontiguousarray(_np(leaf[r])))
            assert np.array_equal(exp, _np(leaves[r])), "replayed leaf states differ"

    def _mcts_expand_and_backprop_dense_priors_batch(self, a, out):
        B, T = int(a[23]), int(a[24])
        for js, local in self._tree_blocks(a, B):
            r = self._rows(T, B, local)
            cq, leaf, st, lm, nl, pri, res, vals, vl, vlen = [np.ascontiguousarray(_np(x[r])) for x in a[13:23]]
            # the leaves' legal lists and results from the oracle's own engine
            om, on, _, _ = self.m.o.batch_legal_features_actions(st, want_features=False, want_actions=False)
            assert np.array_equal(om, lm) and np.array_equal(on, nl), "leaf legal lists differ"
            assert np.array_equal(st[:, 3415].astype(np.int32), res), "leaf results differ"
            self.m.expand_backprop_dense(self._sub(js), cq, leaf, st, om, on, pri, res, vals, vl, vlen,
                                         float(a[26]))


    def _wave_run(self, plan, a):
        roots, active, rnodes, slots = a[:4]
        C, max_root, c_puct, W = int(a[4]), int(a[5]), float(a[6]), int(a[7])
        det, sigma, qp = bool(a[8]), float(a[9]), float(a[10])
        B = plan.B
        T = W * C * B
        first = (plan.tree_base() - self.base) // (4 * self.M)
        for js, local in self._blocks(first, B):
            g = self.torch.tensor(local, device="cuda")
            r = self._rows(T, B, local)
            sub = self._sub(js)
            exp = self.m.select_slots(sub, _np(active[g]), _np(rnodes[g]), np.ascontiguousarray(_np(slots[g])),
                                      max_root, c_puct, W, det, sigma, qp)
            b = {k: np.ascontiguousarray(_np(getattr(plan, k)[:T][r])) for k in (
                "leaf_idx", "move_paths", "path_lens", "vl_paths", "vl_lens", "leaf_states", "results",
                "legal_moves", "num_legal", "priors", "values", "child_q")}
            exp = dict(zip(("leaf_idx", "move_paths", "path_lens", "vl_paths", "vl_lens"), exp))
            for k in ("leaf_idx", "path_lens", "vl_lens"):
                assert np.array_equal(exp[k], b[k]), f"native wave: select output {k} differs"
            # the wave writes each path row up to its recorded length (its readers stop there)
            depth = np.arange(exp["vl_paths"].shape[1])[None, :]
            rec = depth < b["path_lens"][:, None]
            assert np.array_equal(exp["move_paths"][rec], b["move_paths"][rec]), "native wave: move paths differ"
            rec = depth < b["vl_lens"][:, None]
            assert np.array_equal(exp["vl_paths"][rec], b["vl_paths"][rec]), "native wave: node paths differ"
            st = np.zeros((len(r), 3424), np.uint8)
            self.m.replay(np.ascontiguousarray(_np(roots[g])), st, b["move_paths"], b["path_lens"], b["leaf_idx"])
            assert np.array_equal(st, b["leaf_states"]), "native wave: replayed leaf states differ"
            om, on, _, _ = self.m.o.batch_legal_features_actions(st, want_features=False, want_actions=False)
            listed = np.arange(om.shape[1])[None, :] < on[:, None]  # the wave writes each list up to its length
            assert np.array_equal(on, b["num_legal"]) and np.array_equal(om[listed], b["legal_moves"][listed]), \
                "native wave: leaf legal lists differ"
            assert np.array_equal(st[:, 3415].astype(np.int32), b["results"]), "native wave: leaf results differ"
            self.m.expand_backprop_dense(sub, b["child_q"], b["leaf_idx"], st, om, on, b["priors"], b["results"],
                                         b["values"], b["vl_paths"], b["vl_lens"], qp)


def expected_sims(n_legal, n_reserve):
    """Simulations the four halving rounds give a searched game with n_legal
    legal moves, n_reserve of them queen-surround reserve moves
    (fnn_mcts_orchestrator.py:384-444,650-711).  The candidate row is
    [6 reserve columns, -1 padded | 16 fill columns by prior][:16]: the fill
    ranks every slot, the reserve slots and illegal slots at -1e30, so after
    the n - r other legal moves it continues with the reserve slots (lowest
    slot first on ties), which are legal and so considered twice.  Round 0
    therefore has r + min(10, n) valid candidate columns (r = min(6,
    n_reserve)); 1,024 simulations per round over 16, 8, 4, 2 columns;
    survivors halve."""
    r = np.minimum(6, n_reserve)
    v = np.where(n_legal > 0, r + np.minimum(K - 6, n_legal), 0)
    total, C = np.zeros_like(n_legal), K
    for _ in range(4):
        total = total + (1024 // C) * v
        v = np.where(v > 0, np.minimum(C // 2, np.maximum(1, v // 2)), 0)
        C //= 2
    return total


def check_invariants(tree, sims, max_ends, root_legal, root_n, actions):
    """The tree invariants above, on every game's used node prefix (on the GPU)."""
    import torch
    cnt = tree["node_count"].long()
    Mu = int(cnt.max().item())
    node = torch.arange(Mu, device="cuda")[None, :]
    used = node < cnt[:, None]
    vc = tree["visit_count"][:, :Mu].long()
    fc = tree["first_child"][:, :Mu].long()
    nc = tree["num_children"][:, :Mu].long()
    pa = tree["parent_idx"][:, :Mu].long()
    it = tree["is_terminal"][:, :Mu]
    tv = tree["total_value"][:, :Mu]
    assert (tree["root_node"] == 0).all()
    assert not ((fc == -2) & used).any(), "a node left in the expanding state"
    expanded = (fc >= 0) & used
    assert torch.equal((nc * expanded).sum(1) + 1, cnt), "node_count != 1 + children of expanded nodes"
    assert ((fc >= 1) & (fc + nc <= cnt[:, None]) | ~expanded).all(), "child range outside the used prefix"
    assert ((nc == 0) | expanded | ~used).all()
    child = used & (node > 0)
    assert (pa[:, 0] == -1).all() and ((pa >= 0) & (pa < cnt[:, None]) | ~child).all()
    p = pa.clamp(min=0)
    pfc, pnc = fc.gather(1, p), nc.gather(1, p)
    assert ((pfc <= node) & (node < pfc + pnc) | ~child).all(), "a node outside its parent's child range"
    csum = torch.zeros_like(vc).scatter_add_(1, p, torch.where(child, vc, torch.zeros_like(vc)))
    assert torch.equal(vc[:, 0], csum[:, 0]), "root visits != sum of its children's"
    assert torch.equal(vc[:, 0].cpu(), torch.from_numpy(sims).long()), "root visits != scheduled simulations"
    ends = vc - csum
    inner = expanded & (node > 0)
    max_ends = torch.as_tensor(max_ends, device="cuda").reshape(-1, 1)
    assert ((ends >= 1) & (ends <= max_ends) | ~inner).all(), "expanded node ended outside [1, W] simulations"
    assert (expanded | ~(used & (vc > 0) & (it == 0) & (node > 0))).all(), "visited non-terminal leaf unexpanded"
    assert (tree["virtual_q_penalty"][:, :Mu][used] == 0).all()
    assert ((tv.abs() <= vc.float() + 1e-3) | ~used).all(), "|W| > N: a virtual loss left over"
    term = (it != 0) & used
    tval = tree["terminal_value"][:, :Mu][term]
    assert ((tval == 1) | (tval == -1) | (tval == 0)).all() and (fc[term] == -1).all()
    # root children: the legal list in order, with the reference's action indices
    searched = torch.from_numpy(sims > 0).cuda()
    nmax = int(root_n.max().item())
    slot = torch.arange(nmax, device="cuda")[None, :]
    live = (slot < root_n[:, None].long()) & searched[:, None]
    idx = (fc[:, :1] + slot).clamp(0, Mu - 1)
    mb = tree["move_bytes"][:, :Mu][torch.arange(GAMES, device="cuda")[:, None], idx]
    assert torch.equal(mb[live], root_legal[:, :nmax][live])
    assert torch.equal(tree["action_idx"][:, :Mu].gather(1, idx)[live], actions[:, :nmax][live])
    assert torch.equal(nc[:, 0][searched], root_n.long()[searched])


def _run(monkeypatch, wave_parallel, roots, plies=1, mask=0):
    import torch
    from hive_neuralnet_amd import hive_gpu
    from hive_neuralnet_amd.fnn import seeded_large
    from hive_neuralnet_amd.orchestrator import FNNMCTSConfig, FNNMCTSOrchestrator
    from oracle.orchestrator import SearchPlyOracle
    seed = 0x5EED
    net = seeded_large(seed)
    cfg = FNNMCTSConfig(num_simulations=SIMS, max_num_considered_actions=K, batch_size=GAMES,
                        max_tree_nodes=MAX_NODES, wave_parallel=wave_parallel)
    orch = FNNMCTSOrchestrator(net, cfg)
    orch.use_graphs = False
    ext = orch.ext
    if roots == "empty":
        states = ext.create_initial_states(GAMES, mask)
    else:
        states, _ = hive_gpu.random_positions(GAMES, mask, 120, seed + 5)
    torch.manual_seed(seed + 1)
    np.random.seed(seed & 0xFFFF)
    tree = orch._alloc_tree(GAMES)
    sh = SliceShadow(orch, tree, monkeypatch)
    sh.root_base = states.data_ptr()
    active = torch.ones((GAMES,), dtype=torch.bool, device="cuda")
    for ply in range(plies):
        print(f"c5 full: waves={'schedule' if wave_parallel else 1} roots={roots} ply {ply}", flush=True)
        legal, nl = ext.generate_legal_moves_batch(states, GAMES)
        actions = ext.legal_moves_to_actions_batch(states, legal, nl, GAMES)
        wins = _np(orch._find_immediate_wins(states, legal, nl, GAMES)) >= 0
        # reserve moves from the numpy restatement (oracle/orchestrator.py)
        qual = SearchPlyOracle(cfg).qualifying(_np(states), _np(legal), _np(nl))
        r = orch.search_ply(states, tree, active)
        torch.cuda.synchronize()
        sh.check(f"ply {ply}")
        searched = _np(r.has_actions) & ~wins
        sims = expected_sims(np.where(searched, _np(r.num_legal), 0), qual.sum(1))
        assert r.simulations > 0 and int(sims.max()) > 0
        got = _np(r.slot_visits).sum(1)
        want = np.where(wins & _np(r.has_actions), SIMS, sims)
        bad = np.nonzero(got != want)[0]
        diag = os.environ.get("HIVE_TEST_DIAG_DIR")  # where to leave the failing games' data, if anywhere
        if bad.size and diag:
            os.makedirs(diag, exist_ok=True)
            np.savez(os.path.join(diag, "c5_diag.npz"), bad=bad, got=got, want=want, n=_np(r.num_legal),
                     qual=qual.sum(1), wins=wins, has=_np(r.has_actions), sv=_np(r.slot_visits)[bad],
                     states=_np(states)[bad], chosen=_np(r.chosen_slot))
        assert bad.size == 0, (f"{bad.size} games: " + "; ".join(
            f"g{g} n={_np(r.num_legal)[g]} reserve={qual.sum(1)[g]} win={wins[g]} got={got[g]} want={want[g]}"
            for g in bad[:12]))
        # a wave puts W simulations of each candidate column into its root child's
        # subtree; a reserve slot held twice (see expected_sims) doubles that
        n_, r_ = np.where(searched, _np(r.num_legal), 0), np.minimum(6, qual.sum(1))
        twice = (r_ > 0) & (n_ - r_ < K - 6)
        check_invariants(tree, sims, (16 if wave_parallel else 1) * np.where(twice, 2, 1), legal, nl, actions)
        assert sh.calls["mcts_expand_and_backprop_dense_priors_batch"] > 0
        orch.apply_and_rebase(states, tree, r)
        active &= ext.check_results_batch(states, GAMES) == 0
        sh.sync()
    return orch, sh


def test_c5_schedule_midgame_roots_two_ranges(monkeypatch):
    orch, sh = _run(monkeypatch, True, "midgame")
    assert orch.max_game_parts == 2  # the default split ran: two game ranges on two streams
    # 4 rounds x 32 waves, each wave shadowed in both ranges
    assert sh.calls["mcts_select_with_root_slots_batch"] == 2 * 128


def test_c5_one_simulation_per_wave_midgame_roots(monkeypatch):
    orch, sh = _run(monkeypatch, False, "midgame")
    assert orch.max_game_parts == 1  # 8,192-row waves stay on one range
    assert sh.calls["mcts_select_with_root_slots_batch"] == 64 + 128 + 256 + 512


def test_c5_schedule_empty_board_two_plies(monkeypatch):
    _run(monkeypatch, True, "empty", plies=2)
