"""Training-time encoder path and device replay storage on the GPU
(FNNTrainer._build_forward_batch, FNNReplayBuffer counterparts)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("mask,max_ply", [(0, 120), (7, 150)])
def test_build_forward_batch_matches_oracle(oracle, mask, max_ply):
    """A 2,048-position training batch: root features, then the features of every
    legal successor in (root, slot) order, bit-exact with the oracle; with cached
    f16 root features the roots are the f16 rounding of the same values."""
    from hive_neuralnet_amd import hive_gpu
    from hive_neuralnet_amd.replay import build_forward_batch
    ext = hive_gpu.load_extension()
    B = 2048
    states, _ = hive_gpu.random_positions(B, mask, max_ply, 91 + mask)
    root, succ, a2r, nact = build_forward_batch(ext, states, B)
    st = _np(states)
    om, on, of, _ = oracle.batch_legal_features_actions(st)
    assert np.array_equal(_np(nact), on.astype(np.int64))
    assert np.array_equal(_np(root).view(np.uint32), of.view(np.uint32))
    want_a2r = np.repeat(np.arange(B), on)
    mi = np.concatenate([np.arange(k) for k in on])
    assert np.array_equal(_np(a2r), want_a2r)
    want_succ = oracle.batch_successor_features(st, om, want_a2r, mi)
    assert np.array_equal(_np(succ).view(np.uint32), want_succ.view(np.uint32))
    legal, nl, feat = ext.generate_legal_moves_and_fnn_features_batch(states, B)
    r2, s2, a2, n2 = build_forward_batch(ext, states, B, nl, feat.half(), legal)
    assert np.array_equal(_np(r2), of.astype(np.float16).astype(np.float32))
    assert np.array_equal(_np(s2).view(np.uint32), want_succ.view(np.uint32))


def test_replay_buffer_ring_and_sampling():
    import torch
    from hive_neuralnet_amd.fnn import seeded_large
    from hive_neuralnet_amd.orchestrator import FNNMCTSConfig, FNNMCTSOrchestrator
    from hive_neuralnet_amd.replay import FNNReplayBuffer
    torch.manual_seed(5)
    np.random.seed(5)
    games = FNNMCTSOrchestrator(seeded_large(4), FNNMCTSConfig(num_simulations=16, batch_size=6,
                                                              max_tree_nodes=2048, max_game_length=10)).self_play_batch()
    ex = [e for g in games for e in g]
    buf = FNNReplayBuffer(max_size=25, merge_opening_value_examples=False)
    buf.add_examples(ex[:20])
    buf.add_examples(ex[20:])  # wraps: the ring holds the last 25 examples
    assert len(buf) == min(25, len(ex))
    t = buf._t
    for i in range(max(0, len(ex) - 25), len(ex)):  # example i sits in ring slot i % 25
        s, e = i % 25, ex[i]
        n = e.policy_target.shape[0]
        assert np.array_equal(_np(t["states"][s]), e.state_bytes)
        assert np.array_equal(_np(t["policy"][s][:n]), e.policy_target.astype(np.float16))
        assert int(t["num_actions"][s]) == n and float(t["values"][s, 0]) == e.value_target
    # cached root features = f16 of the engine's features of the stored state
    legal, nl, feat = buf.ext.generate_legal_moves_and_fnn_features_batch(t["states"], 25)
    assert torch.equal(t["root_features"], feat.half()) and torch.equal(t["legal_moves"], legal)
    torch.manual_seed(9)
    b = buf.sample_batch(64, device="cuda")
    torch.manual_seed(9)
    idx = torch.randint(0, 25, (64,), device="cuda", dtype=torch.int64)
    assert torch.equal(b.state_bytes, t["states"][idx]) and torch.equal(b.policy_targets, t["policy"][idx].float())
    assert b.root_features.dtype == torch.float32 and b.legal_moves.shape == (64, 256, 6)
