"""FNN leaf evaluator: the reference's HiveFNN network (hive_fnn/fnn_network.py).

Same layers, construction order and parameter names (fc1, ln1, fc2,
value_fc, action_fc1, action_fc2), so a reference state dict loads as is and
seeded random initialisation (torch.manual_seed + PyTorch's default Linear /
LayerNorm init) gives the same weights:

    encode(x)            = fc2(LayerNorm(sigmoid(fc1 x)))        (fnn_network.py:175-187)
    value_head(e)        = tanh(value_fc e)                      (:189-199)
    score_actions(r, s)  = action_fc2(sigmoid(action_fc1 [r | s]))  (:204-220)

`large` = 64/64/64 -> 20,546 parameters at the 122-dim input.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn

FEAT_DIM = 122


@dataclass
class FNNConfig:
    feat_dim: int = FEAT_DIM
    hidden_dim: int = 64
    embed_dim: int = 64
    action_hidden: int = 64

    @classmethod
    def small(cls) -> "FNNConfig":
        return cls(hidden_dim=8, embed_dim=8, action_hidden=8)

    @classmethod
    def medium(cls) -> "FNNConfig":
        return cls(hidden_dim=32, embed_dim=32, action_hidden=32)

    @classmethod
    def large(cls) -> "FNNConfig":
        return cls(hidden_dim=64, embed_dim=64, action_hidden=64)


class HiveFNN(nn.Module):
    def __init__(self, config: FNNConfig | None = None) -> None:
        super().__init__()
        self.config = config or FNNConfig.large()
        self.config.feat_dim = FEAT_DIM
        c = self.config
        self.fc1 = nn.Linear(c.feat_dim, c.hidden_dim)
        self.ln1 = nn.LayerNorm(c.hidden_dim)
        self.fc2 = nn.Linear(c.hidden_dim, c.embed_dim)
        self.value_fc = nn.Linear(c.embed_dim, 1)
        self.action_fc1 = nn.Linear(c.embed_dim * 2, c.action_hidden)
        self.action_fc2 = nn.Linear(c.action_hidden, 1)

    def load_state_dict(self, state_dict, strict: bool = True, assign: bool = False):
        """Loads checkpoints whose fc1 was trained on a different feature count
        (fnn_network.py:74-94): the overlapping block of fc1.weight is kept and the
        rest drawn from N(0, 1e-3)."""
        state = dict(state_dict)
        cur = self.fc1.weight
        old = state.get("fc1.weight")
        if old is not None and old.shape != cur.shape:
            grown = torch.empty_like(cur).normal_(mean=0.0, std=1e-3)
            r, c = min(old.shape[0], cur.shape[0]), min(old.shape[1], cur.shape[1])
            grown[:r, :c] = old[:r, :c].to(grown)
            state["fc1.weight"] = grown
        return super().load_state_dict(state, strict=strict, assign=assign)

    def encode(self, features: torch.Tensor) -> torch.Tensor:
        return self.fc2(self.ln1(torch.sigmoid(self.fc1(features))))

    def value_head(self, embed: torch.Tensor) -> torch.Tensor:
        return torch.tanh(self.value_fc(embed))

    def score_actions(self, root_embed: torch.Tensor, successor_embed: torch.Tensor) -> torch.Tensor:
        x = torch.sigmoid(self.action_fc1(torch.cat([root_embed, successor_embed], dim=1)))
        return self.action_fc2(x).squeeze(-1)

    def forward(self, root_features, successor_features, action_to_root, num_actions):
        """Training forward (fnn_network.py:224-253): (action_logits [N], root_values [B,1])."""
        root_emb = self.encode(root_features)
        root_values = self.value_head(root_emb)
        if action_to_root.shape[0] == 0:
            return root_features.new_zeros((0,)), root_values
        succ_emb = self.encode(successor_features)
        return self.score_actions(root_emb[action_to_root], succ_emb), root_values

    def count_parameters(self) -> int:
        return sum(p.numel() for p in self.parameters() if p.requires_grad)


def seeded_large(seed: int, device: str = "cuda") -> HiveFNN:
    """Random-init `large` network under torch.manual_seed(seed) (the C5 configuration)."""
    torch.manual_seed(seed)
    return HiveFNN(FNNConfig.large()).to(device).eval()
