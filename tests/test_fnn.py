"""FNN leaf evaluator (hive_fnn/fnn_network.py counterpart): structure and math on the CPU."""
import numpy as np
import torch

from hive_neuralnet_amd.fnn import FEAT_DIM, FNNConfig, HiveFNN, seeded_large


def test_parameter_counts_and_names():
    # fnn_network.py:59-71: fc1, ln1, fc2, value_fc, action_fc1, action_fc2
    large = HiveFNN(FNNConfig.large())
    assert FEAT_DIM == 122
    # 122*64+64 + 2*64 + 64*64+64 + 64+1 + 128*64+64 + 64+1
    assert large.count_parameters() == 20546
    assert HiveFNN(FNNConfig.small()).count_parameters() == 122 * 8 + 8 + 16 + 72 + 9 + 16 * 8 + 8 + 9
    assert list(large.state_dict().keys()) == [
        "fc1.weight", "fc1.bias", "ln1.weight", "ln1.bias", "fc2.weight", "fc2.bias", "value_fc.weight",
        "value_fc.bias", "action_fc1.weight", "action_fc1.bias", "action_fc2.weight", "action_fc2.bias"]


def test_seeded_init_is_reproducible():
    a = seeded_large(123, device="cpu")
    b = seeded_large(123, device="cpu")
    c = seeded_large(124, device="cpu")
    for (k, x), (_, y), (_, z) in zip(a.state_dict().items(), b.state_dict().items(), c.state_dict().items()):
        assert torch.equal(x, y), k
    assert not torch.equal(a.fc1.weight, c.fc1.weight)


def test_forward_against_numpy_float64():
    """encode/value/score restated independently in float64 numpy."""
    net = seeded_large(7, device="cpu")
    torch.manual_seed(0)
    for p in net.ln1.parameters():   # non-trivial LayerNorm affine
        p.data.uniform_(-1, 1)
    x = torch.rand(5, FEAT_DIM)
    W = {k: v.double().numpy() for k, v in net.state_dict().items()}
    xd = x.double().numpy()
    h = 1 / (1 + np.exp(-(xd @ W["fc1.weight"].T + W["fc1.bias"])))
    h = (h - h.mean(1, keepdims=True)) / np.sqrt(h.var(1, keepdims=True) + 1e-5)
    h = h * W["ln1.weight"] + W["ln1.bias"]
    e = h @ W["fc2.weight"].T + W["fc2.bias"]
    v = np.tanh(e @ W["value_fc.weight"].T + W["value_fc.bias"])[:, 0]
    a2r = np.array([0, 0, 1, 3, 4])
    s = np.concatenate([e[a2r], e[[1, 2, 3, 4, 0]]], axis=1)
    z = 1 / (1 + np.exp(-(s @ W["action_fc1.weight"].T + W["action_fc1.bias"])))
    logit = (z @ W["action_fc2.weight"].T + W["action_fc2.bias"])[:, 0]
    with torch.no_grad():
        emb = net.encode(x)
        logits, vals = net(x, x[[1, 2, 3, 4, 0]], torch.tensor(a2r), 5)
    np.testing.assert_allclose(emb.numpy(), e, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(vals[:, 0].numpy(), v, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(logits.numpy(), logit, rtol=1e-5, atol=1e-5)


def test_load_state_dict_grows_fc1():
    """A checkpoint trained on fewer features loads: the known block is kept."""
    net = seeded_large(1, device="cpu")
    sd = {k: v.clone() for k, v in net.state_dict().items()}
    sd["fc1.weight"] = sd["fc1.weight"][:, :100].clone()
    other = seeded_large(2, device="cpu")
    other.load_state_dict(sd)
    assert torch.equal(other.fc1.weight[:, :100], net.fc1.weight[:, :100])
    assert other.fc1.weight[:, 100:].abs().max() < 0.01
    assert torch.equal(other.fc2.weight, net.fc2.weight)
