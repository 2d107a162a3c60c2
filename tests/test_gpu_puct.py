"""Plain PUCT self-play (hive_fnn/fnn_puct_orchestrator.py counterpart) on the
GPU: every tree call of real search plies shadowed by the C tree oracle, the
visit-count policy and move choice, and whole games."""
import numpy as np
import pytest

from test_gpu_orchestrator import Shadow, _np

pytestmark = pytest.mark.gpu


def _puct(B, sims, M, seed, **kw):
    from hive_neuralnet_amd.fnn import seeded_large
    from hive_neuralnet_amd.puct import FNNPUCTConfig, FNNPUCTOrchestrator
    return FNNPUCTOrchestrator(seeded_large(seed), FNNPUCTConfig(num_simulations=sims, batch_size=B,
                                                                   max_tree_nodes=M, **kw))


@pytest.mark.parametrize("sims,W,M,mask,max_ply", [(40, 16, 4096, 7, 50), (24, 4, 600, 0, 30)],
                         ids=["w16", "w4-pool-exhaustion"])
def test_puct_ply_tree_calls_match_oracle(monkeypatch, sims, W, M, mask, max_ply):
    import torch
    from hive_neuralnet_amd import hive_gpu
    B = 10
    orch = _puct(B, sims, M, 61, wave_size=W)
    # positions without an immediate win: one in the batch would skip the search of every game
    pool, _ = hive_gpu.random_positions(64, mask, max_ply, 62)
    legal, nl = orch.ext.generate_legal_moves_batch(pool, 64)
    ok = (orch._find_immediate_wins(pool, legal, nl, 64) < 0) & (nl > 0)
    states = pool[torch.nonzero(ok).squeeze(1)[:B]].contiguous()
    assert states.shape[0] == B
    torch.manual_seed(63)
    np.random.seed(63)
    tree = orch._alloc_tree(B)
    sh = Shadow(orch._eval_helper, tree, monkeypatch)
    out = orch.search_ply(states, tree, torch.ones((B,), dtype=torch.bool, device="cuda"),
                          torch.zeros((B,), dtype=torch.int64, device="cuda"))
    assert sh.calls.get("mcts_select_with_root_mask_batch", 0) == (sims + W - 1) // W
    sh.check_tree("end of ply")
    chosen, legal, nl, probs, visits, has = (_np(x) for x in out)
    # the policy is the root children's visit distribution over legal slots
    for i in np.nonzero(has)[0]:
        n = nl[i]
        assert visits[i, n:].sum() == 0 and (probs[i, n:] == 0).all()
        if visits[i].sum() > 0:
            np.testing.assert_allclose(probs[i, :n], visits[i, :n] / visits[i].sum(), rtol=1e-6)
        assert 0 <= chosen[i] < n and probs[i, chosen[i]] > 0


def test_puct_greedy_after_temperature_drop():
    import torch
    from hive_neuralnet_amd import hive_gpu
    B = 6
    orch = _puct(B, 32, 4096, 64)
    pool, _ = hive_gpu.random_positions(64, 0, 40, 65)
    legal, nl = orch.ext.generate_legal_moves_batch(pool, 64)
    ok = (orch._find_immediate_wins(pool, legal, nl, 64) < 0) & (nl > 0)
    states = pool[torch.nonzero(ok).squeeze(1)[:B]].contiguous()
    tree = orch._alloc_tree(B)
    out = orch.search_ply(states, tree, torch.ones((B,), dtype=torch.bool, device="cuda"),
                          torch.full((B,), 25, dtype=torch.int64, device="cuda"))
    chosen, _, _, probs, _, has = (_np(x) for x in out)
    for i in np.nonzero(has)[0]:
        assert chosen[i] == int(np.argmax(probs[i]))


def test_puct_self_play_batch():
    orch = _puct(4, 16, 2048, 66, max_game_length=8, wave_size=8)
    import torch
    torch.manual_seed(67)
    np.random.seed(67)
    games = orch.self_play_batch()
    assert len(games) == 4
    for g in games:
        assert 1 <= len(g) <= 8
        for e in g:
            assert e.state_bytes.shape == (3424,)
            assert abs(float(e.policy_target.sum()) - 1.0) < 1e-5
            assert e.value_target in (-1.0, 0.0, 1.0)
