"""Replay storage and the training-time encoder path of the FNN line, on the
MI355X engine: counterparts of hive_fnn/fnn_replay_buffer.py (FNN fields)
and FNNTrainer._build_forward_batch (hive_fnn/fnn_trainer.py:531-580).

Storage keeps the reference's record format -- state bytes [N, 3424] u8,
policy [N, 256] f16 over the legal list, action counts, value target / masks
/ weights, and (cache_root_features) the root features [N, 122] f16 with the
legal list [N, 256, 6] u8 computed by the engine when examples are added --
resident in device memory (a 288 GB device holds millions of records), so
sampling and the forward-batch build never cross PCIe.  The hybrid/token
feature caches of the reference buffer belong to the transformer line and
are not kept.

build_forward_batch returns (root features, successor features, action_to_root,
num_actions) for a batch of state bytes exactly as the trainer's method: the
root features and legal lists (cached or generated), then the 122 features of
every legal successor, rows in (root, slot) order.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import hive_gpu
from .orchestrator import FNNTrainingExample

_OFF_TURN = 3412
FEAT_DIM = 122


@dataclass
class FNNTrainingBatch:  # fnn_replay_buffer.py:34-49 (FNN fields)
    state_bytes: torch.Tensor
    policy_targets: torch.Tensor
    num_actions: torch.Tensor
    value_targets: torch.Tensor
    policy_mask: torch.Tensor
    value_mask: torch.Tensor
    value_weights: torch.Tensor
    root_features: torch.Tensor | None = None
    legal_moves: torch.Tensor | None = None


def build_forward_batch(ext, state_bytes: torch.Tensor, batch_size: int, num_actions: torch.Tensor | None = None,
                        cached_root_features: torch.Tensor | None = None,
                        cached_legal_moves: torch.Tensor | None = None):
    """FNNTrainer._build_forward_batch (fnn_trainer.py:531-580): (root_features
    [B, 122], successor_features [N, 122], action_to_root [N] int64,
    num_actions [B] int64)."""
    if cached_root_features is not None and cached_legal_moves is not None:
        if num_actions is None:
            raise ValueError("Cached legal moves require cached action counts")
        root_features = cached_root_features.float()
        legal_moves = cached_legal_moves
        num_actions = num_actions.to(torch.int64)
    else:
        legal_moves, num_legal, root_features = ext.generate_legal_moves_and_fnn_features_batch(state_bytes, batch_size)
        num_actions = num_legal.to(torch.int64)
    dev = state_bytes.device
    # rows in (root, slot) order: one host read of the row count, the row map
    # built on the device
    counts = num_actions.clamp(0, legal_moves.shape[1])
    total = int(counts.sum().item())
    if total == 0:
        return root_features, root_features[:0], torch.zeros((0,), dtype=torch.int64, device=dev), num_actions
    roots = torch.arange(batch_size, device=dev, dtype=torch.int64)
    action_to_root = torch.repeat_interleave(roots, counts, output_size=total)
    starts = torch.cumsum(counts, 0) - counts
    move_indices = torch.arange(total, device=dev, dtype=torch.int64) - starts[action_to_root]
    succ = ext.fnn_successor_features_batch(state_bytes, legal_moves, action_to_root, move_indices, total)
    return root_features, succ, action_to_root, num_actions


class FNNReplayBuffer:
    """Ring buffer of FNN training examples in device memory
    (FNNReplayBuffer, fnn_replay_buffer.py:100-660, FNN fields)."""

    def __init__(self, max_size: int = 100_000, *, device: torch.device | str | None = None,
                 cache_root_features: bool = True, merge_opening_value_examples: bool = True,
                 opening_value_merge_plies: int = 4) -> None:
        self.max_size = int(max_size)
        self.device = torch.device(device or "cuda")
        self.cache_root_features = bool(cache_root_features)
        self.merge_opening_value_examples = bool(merge_opening_value_examples)
        self.opening_value_merge_plies = max(0, int(opening_value_merge_plies))
        self.ext = hive_gpu.load_extension()
        self.max_actions = int(self.ext.MAX_LEGAL_MOVES)
        self._size = 0
        self._next_idx = 0
        self._uniform_weights = True
        self._t: dict[str, torch.Tensor] | None = None

    def __len__(self) -> int:
        return self._size

    def _allocate(self, state_size: int) -> None:
        N, d = self.max_size, self.device
        self._t = {
            "states": torch.empty((N, state_size), dtype=torch.uint8, device=d),
            "policy": torch.zeros((N, self.max_actions), dtype=torch.float16, device=d),
            "num_actions": torch.zeros((N,), dtype=torch.int64, device=d),
            "values": torch.zeros((N, 1), dtype=torch.float32, device=d),
            "policy_mask": torch.zeros((N, 1), dtype=torch.float32, device=d),
            "value_mask": torch.zeros((N, 1), dtype=torch.float32, device=d),
            "weights": torch.ones((N,), dtype=torch.float32, device=d),
            "value_weights": torch.ones((N, 1), dtype=torch.float32, device=d),
        }
        if self.cache_root_features:
            self._t["root_features"] = torch.zeros((N, FEAT_DIM), dtype=torch.float16, device=d)
            self._t["legal_moves"] = torch.zeros((N, self.max_actions, 6), dtype=torch.uint8, device=d)

    @staticmethod
    def _state_turn(state_bytes: np.ndarray) -> int:
        return int(state_bytes[_OFF_TURN]) | (int(state_bytes[_OFF_TURN + 1]) << 8)

    def _compact_opening_value_examples(self, examples):  # fnn_replay_buffer.py:309-353
        if not self.merge_opening_value_examples:
            return examples
        return compact_opening_value_examples(examples, self.opening_value_merge_plies)

    def add_examples(self, examples) -> None:
        if not examples:
            return
        examples = self._compact_opening_value_examples(list(examples))
        if self._t is None:
            self._allocate(int(examples[0].state_bytes.shape[0]))
        # ring order: the reference's two slices (:280-304); an add longer than
        # the buffer keeps wrapping (the reference's second slice would overflow)
        count, off, pos = len(examples), 0, self._next_idx
        while off < count:
            n = min(count - off, self.max_size - pos)
            self._write_chunk(examples[off: off + n], pos)
            off += n
            pos = (pos + n) % self.max_size
        self._next_idx = pos
        self._size = min(self.max_size, self._size + count)

    def _write_chunk(self, examples, lo: int) -> None:  # fnn_replay_buffer.py:355-531
        B = len(examples)
        t = self._t
        states = np.stack([ex.state_bytes for ex in examples]).astype(np.uint8, copy=False)
        policy = np.zeros((B, self.max_actions), np.float16)
        num = np.zeros((B,), np.int64)
        rest = np.zeros((B, 5), np.float32)  # value, policy mask, value mask, surprise weight, value weight
        for i, ex in enumerate(examples):
            n = int(ex.policy_target.shape[0])
            policy[i, :n] = ex.policy_target.astype(np.float16, copy=False)
            num[i] = n
            rest[i] = (ex.value_target, float(ex.use_for_policy), float(ex.use_for_value),
                       ex.surprise_weight, ex.value_weight)
        self._uniform_weights = self._uniform_weights and bool((rest[:, 3] == 1.0).all())
        dst = slice(lo, lo + B)
        d = self.device
        st = torch.from_numpy(states).to(d)
        t["states"][dst] = st
        t["policy"][dst] = torch.from_numpy(policy).to(d)
        t["num_actions"][dst] = torch.from_numpy(num).to(d)
        r = torch.from_numpy(rest).to(d)
        t["values"][dst] = r[:, 0:1]
        t["policy_mask"][dst] = r[:, 1:2]
        t["value_mask"][dst] = r[:, 2:3]
        t["weights"][dst] = r[:, 3]
        t["value_weights"][dst] = r[:, 4:5]
        if self.cache_root_features:
            legal, _, feat = self.ext.generate_legal_moves_and_fnn_features_batch(st, B)
            t["root_features"][dst] = feat.to(torch.float16)
            t["legal_moves"][dst] = legal

    def _sample_indices(self, batch_size: int) -> torch.Tensor:  # :533-543
        if self._uniform_weights:
            return torch.randint(0, self._size, (batch_size,), device=self.device, dtype=torch.int64)
        w = self._t["weights"][: self._size]
        return torch.multinomial(w / w.sum(), batch_size, replacement=True)

    def sample_batch(self, batch_size: int, *, device: torch.device | None = None,
                     non_blocking: bool = False) -> FNNTrainingBatch:
        if self._size == 0:
            raise ValueError("Cannot sample from an empty replay buffer")
        t = self._t
        idx = self._sample_indices(batch_size)
        sel = lambda k: t[k].index_select(0, idx)  # noqa: E731
        b = FNNTrainingBatch(sel("states"), sel("policy").float(), sel("num_actions"), sel("values"),
                             sel("policy_mask"), sel("value_mask"), sel("value_weights"),
                             sel("root_features").float() if self.cache_root_features else None,
                             sel("legal_moves") if self.cache_root_features else None)
        if device is not None and torch.device(device) != self.device:
            b = FNNTrainingBatch(*[None if x is None else x.to(device, non_blocking=non_blocking)
                                   for x in b.__dict__.values()])
        return b


def compact_opening_value_examples(examples, plies: int):
    """_compact_opening_value_examples (fnn_replay_buffer.py:309-353): value
    examples of an opening position (turn < plies) that occurs more than once
    in the list are merged -- each occurrence keeps its policy example with
    use_for_value off, and one value-only example carries the weight-averaged
    value target with the summed weight (the count when the weights sum to 0),
    appended after the examples that were not grouped, groups in order of
    first occurrence."""
    if plies <= 0:
        return examples
    turn = lambda sb: int(sb[_OFF_TURN]) | (int(sb[_OFF_TURN + 1]) << 8)  # noqa: E731
    merged, groups = [], {}
    for ex in examples:
        if not ex.use_for_value or turn(ex.state_bytes) >= plies:
            merged.append(ex)
            continue
        groups.setdefault(ex.state_bytes.tobytes(), []).append(ex)
    for grouped in groups.values():
        if len(grouped) == 1:
            merged.append(grouped[0])
            continue
        for ex in grouped:
            merged.append(_replace(ex, use_for_value=False))
        total_w = sum(float(ex.value_weight) for ex in grouped)
        if total_w <= 0.0:
            total_w = float(len(grouped))
        avg = sum(float(ex.value_target) * float(ex.value_weight) for ex in grouped) / total_w
        rep = grouped[0]
        merged.append(FNNTrainingExample(rep.state_bytes, rep.policy_target, float(avg), False, True, float(total_w),
                                         rep.surprise_weight))
    return merged


def _replace(ex: FNNTrainingExample, **kw) -> FNNTrainingExample:
    d = dict(ex.__dict__)
    d.update(kw)
    return FNNTrainingExample(**d)
