"""Root tactical probe (root_tactical_probe_batch, game_logic.cu:290-397) on
the GPU: against the reference's golden vectors, against the C oracle on
seeded random-play positions, and inside the self-play orchestrator
(short_forced_win_probe) against the numpy restatement of a search ply."""
import numpy as np
import pytest

from conftest import load_golden

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().numpy()


def _run(ext, st, lm, nl, pr, flags):
    import torch
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    w, a, f = ext.root_tactical_probe_batch(dev(st), dev(lm), dev(nl), dev(pr), len(st), *[bool(x) for x in flags])
    torch.cuda.synchronize()
    assert w.dtype == torch.int64 and a.dtype == torch.uint8 and f.dtype == torch.uint8
    return _np(w), _np(a), _np(f)


def test_probe_golden_vectors():
    from hive_neuralnet_amd import hive_gpu
    ext = hive_gpu.load_extension()
    g = load_golden("probe")
    for j, flags in enumerate(g["flags"]):
        print("flags", tuple(flags), flush=True)
        w, a, f = _run(ext, g["states"], g["legal"], g["nlegal"], g["priors"], flags)
        assert np.array_equal(w, g["win"][j]), (tuple(flags), np.nonzero(w != g["win"][j])[0][:8])
        assert np.array_equal(f, g["forced"][j]), tuple(flags)
        assert np.array_equal(a, g["allowed"][j]), tuple(flags)


def test_probe_single_roots_part_programs():
    """Every two-move root of the reference vectors ('w2' and 'forced'), each
    probed alone (a batch of one), under all four flag combinations.  The
    grandchild list then holds 256 entries, fewer than many of these roots'
    surviving candidates need (roots 209, 215, 219, 230, 244 and 258 among
    them, by the wave emulator), so those candidates are tested by the part
    programs (k_probe_win2) instead, the path large batches rarely take."""
    from hive_neuralnet_amd import hive_gpu
    ext = hive_gpu.load_extension()
    g = load_golden("probe")
    roots = np.nonzero(np.isin(g["kinds"], ["w2", "forced"]))[0]
    assert {209, 215, 219, 230, 244, 258} <= set(roots.tolist())
    for j, flags in enumerate(g["flags"]):
        for r in roots:
            sl = slice(int(r), int(r) + 1)
            w, a, f = _run(ext, g["states"][sl], g["legal"][sl], g["nlegal"][sl], g["priors"][sl], flags)
            assert w[0] == g["win"][j][r], (tuple(flags), int(r))
            assert f[0] == g["forced"][j][r], (tuple(flags), int(r))
            assert np.array_equal(a[0], g["allowed"][j][r]), (tuple(flags), int(r))


@pytest.mark.parametrize("mask,max_ply,seed", [(0, 150, 41), (7, 150, 42), (0, 300, 43)])
def test_probe_matches_oracle(oracle, mask, max_ply, seed):
    """4,096 GPU-generated positions per case (about one in six has a gate open),
    priors in steps of 1/8 (ties), every stage enabled."""
    from hive_neuralnet_amd import hive_gpu
    ext = hive_gpu.load_extension()
    B = 4096
    print("case", mask, max_ply, seed, flush=True)
    states, _ = hive_gpu.random_positions(B, mask, max_ply, seed)
    legal, nl = ext.generate_legal_moves_batch(states, B)
    st, lm, n = _np(states), _np(legal), _np(nl)
    pr = (np.random.default_rng(seed).integers(0, 8, size=(B, 256)) / 8.0).astype(np.float32)
    w, a, f = _run(ext, st, lm, n, pr, (1, 1, 1))
    ow, oa, of = oracle.batch_root_tactical_probe(st, lm, n, pr)
    assert np.array_equal(w, ow), np.nonzero(w != ow)[0][:8]
    assert np.array_equal(f, of)
    assert np.array_equal(a, oa)
    assert (w >= 0).sum() > 20 and (a[np.arange(256)[None, :] < n[:, None]] == 0).any()


def test_probe_edge_cases(oracle):
    """Empty batch, finished games, rows with no legal move and num_legal
    beyond 256 (clamped)."""
    import torch
    from hive_neuralnet_amd import hive_gpu
    ext = hive_gpu.load_extension()
    w, a, f = ext.root_tactical_probe_batch(torch.zeros((0, 3424), dtype=torch.uint8, device="cuda"),
                                            torch.zeros((0, 256, 6), dtype=torch.uint8, device="cuda"),
                                            torch.zeros((0,), dtype=torch.int32, device="cuda"),
                                            torch.zeros((0, 256), dtype=torch.float32, device="cuda"), 0)
    assert w.shape == (0,) and a.shape == (0, 256) and f.shape == (0,)
    g = load_golden("probe")
    st, lm, nl, pr = (g[k][:40].copy() for k in ("states", "legal", "nlegal", "priors"))
    st[0, 3415] = 1          # finished game
    nl[1] = 0                # no legal move
    nl[2] = 300              # clamped to 256
    w, a, f = _run(ext, st, lm, nl, pr, (1, 1, 1))
    ow, oa, of = oracle.batch_root_tactical_probe(st, lm, nl, pr)
    assert np.array_equal(w, ow) and np.array_equal(a, oa) and np.array_equal(f, of)
    assert w[0] == -1 and w[1] == -1 and not a[1].any() and a[0, : nl[0]].all()


def test_orchestrator_probe_matches_numpy(monkeypatch):
    """search_ply with short_forced_win_probe on twelve games drawn from the
    probe fixture (immediate wins, two-move wins, screened lists, forced
    random moves) against oracle/orchestrator.py fed the recorded network
    outputs and random draws."""
    import torch
    from hive_neuralnet_amd.fnn import seeded_large
    from hive_neuralnet_amd.orchestrator import FNNMCTSConfig, FNNMCTSOrchestrator
    from mcts_driver import tree_equal
    from oracle.orchestrator import SearchPlyOracle
    g = load_golden("probe")
    kinds = g["kinds"]
    sel = np.concatenate([np.nonzero(kinds == k)[0][:2] for k in ("w1", "w2", "screened", "forced", "none",
                                                                  "ungated")])
    B = len(sel)
    net = seeded_large(51)
    cfg = FNNMCTSConfig(num_simulations=32, batch_size=B, max_tree_nodes=1 << 14, short_forced_win_probe=True)
    orch = FNNMCTSOrchestrator(net, cfg)
    orch.use_graphs = False  # the recording reads every evaluation on the host
    states = torch.from_numpy(np.ascontiguousarray(g["states"][sel])).cuda()
    torch.manual_seed(52)
    np.random.seed(52)
    tree = orch._alloc_tree(B)
    evals, uniforms, noises = [], [], []
    real_eval, real_rand = orch._eval_states, torch.rand
    ext = orch.ext
    real_noise = ext.mcts_apply_root_noise

    def rec_eval(*a, **k):
        out = real_eval(*a, **k)
        evals.append(tuple(_np(x).copy() for x in out))
        return out

    def rec_rand(*a, **k):
        out = real_rand(*a, **k)
        uniforms.append(_np(out).copy())
        return out

    def rec_noise(*a):
        noises.append(_np(a[12]).copy())
        return real_noise(*a)

    monkeypatch.setattr(orch, "_eval_states", rec_eval)
    from mcts_driver import record_wave_evaluations
    record_wave_evaluations(monkeypatch, evals)
    monkeypatch.setattr(torch, "rand", rec_rand)
    monkeypatch.setattr(ext, "mcts_apply_root_noise", rec_noise, raising=False)
    t0 = {k: _np(v).copy() for k, v in tree.items()}
    st = _np(states).copy()
    r = orch.search_ply(states, tree, torch.ones((B,), dtype=torch.bool, device="cuda"))
    fr = _np(r.forced_random)
    assert fr.sum() == 2 and len(uniforms) == 2
    ref = SearchPlyOracle(orch.config)
    legal, n, _, _ = ref.o.batch_legal_features_actions(st, want_features=False, want_actions=False)
    chosen, probs, visits = ref.run(t0, st, np.ones(B, bool), legal, n, evals[0], uniforms[0], noises[0], evals[1:],
                                    forced_uniforms=uniforms[1])
    assert np.array_equal(chosen, _np(r.chosen_slot))
    assert np.array_equal(visits, _np(r.slot_visits))
    np.testing.assert_allclose(probs, _np(r.policy), atol=2e-6, rtol=0)
    assert tree_equal(t0, {k: _np(v) for k, v in tree.items()}) == []
    assert (_np(r.policy)[fr] == 0).all() and (_np(r.chosen_slot)[fr] < n[fr]).all()
