"""Plain PUCT self-play over the MI355X engine: the counterpart of the
reference's FNNPUCTOrchestrator (hive_fnn/fnn_puct_orchestrator.py).

Per ply (self_play_batch, :140-297): legal lists + root features,
immediate-win override, leaf evaluation of every legal successor with the FNN
(the Gumbel orchestrator's fused path), root expansion and Dirichlet noise,
waves of root-mask PUCT simulations with every legal root child alive
(:340-384), visit-count policy (uniform when nothing was visited), greedy or
sampled move by move number, apply + rebase.

Deliberate differences from the reference:
  * the tree tensors go to the kernels in the extension's argument order; the
    reference passes virtual_q_penalty and parent_idx swapped
    (fnn_puct_orchestrator.py:110-117 against bindings.cpp:392-436), so its
    kernels read parent indices as float penalties (int -1 is a float NaN),
    and this extension would reject that call (dtype check);
  * per-game Python loops (root child statistics, rebase) are vectorised;
  * the tree kernels apply each game's simulations in simulation order.
Quirks kept: when any game of the batch has an immediate win no game
searches that ply, and games without a win get an all-zero policy and play
slot 0 (:186-197,224-236).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import hive_gpu
from .fnn import HiveFNN
from .orchestrator import FNNMCTSConfig, FNNMCTSOrchestrator, FNNTrainingExample

_OFF_TURN = 3412


@dataclass
class FNNPUCTConfig:  # fnn_puct_orchestrator.py:24-41 (same fields and defaults)
    num_simulations: int = 128
    c_puct: float = 1.25
    temperature: float = 1.0
    temperature_drop_move: int = 20
    batch_size: int = 128
    max_game_length: int = 300
    expansion_mask: int = 0
    wave_size: int = 16
    dirichlet_alpha: float = 0.3
    dirichlet_epsilon: float = 0.25
    max_tree_nodes: int = 65536
    final_value_ply_count: int = 3
    final_value_weight: float = 2.0
    rebase_tree_each_move: bool = True


class FNNPUCTOrchestrator:
    """Plain PUCT MCTS for the FNN backbone."""

    def __init__(self, net: HiveFNN, config: FNNPUCTConfig | None = None) -> None:
        self.ext = hive_gpu.load_extension()
        self.config = config or FNNPUCTConfig()
        self.net = net
        self._max_nodes = int(self.config.max_tree_nodes)
        self._max_legal = int(self.ext.MAX_LEGAL_MOVES)
        c = self.config
        self._eval_helper = FNNMCTSOrchestrator(net, FNNMCTSConfig(
            num_simulations=c.num_simulations, batch_size=c.batch_size, max_game_length=c.max_game_length,
            expansion_mask=c.expansion_mask, wave_size=c.wave_size, dirichlet_alpha=c.dirichlet_alpha,
            dirichlet_epsilon=c.dirichlet_epsilon, max_tree_nodes=c.max_tree_nodes,
            rebase_tree_each_move=c.rebase_tree_each_move))
        self._slot_idx = torch.arange(self._max_legal, device="cuda", dtype=torch.int64).unsqueeze(0)

    # ---- tree ----------------------------------------------------------
    def _alloc_tree(self, B: int) -> dict:
        return self._eval_helper._alloc_tree(B)

    def _tree_args(self, tree: dict) -> list:
        return self._eval_helper._tree_args(tree)

    def _eval_states(self, states, legal_moves, num_legal, total, root_features=None):
        return self._eval_helper._eval_states(states, legal_moves, num_legal, total, root_features)

    def _find_immediate_wins(self, states, legal_moves, num_legal, total):
        return self._eval_helper._find_immediate_wins(states, legal_moves, num_legal, total)

    def _expand_root_if_needed(self, tree, states, legal, nl, priors, child_q, game_active, B):  # :300-316
        self._eval_helper._expand_root_if_needed(tree, states, legal, nl, priors, child_q, game_active, B)

    def _apply_root_dirichlet(self, tree, B, active):  # :318-339
        cfg = self.config
        nc = tree["num_children"][torch.arange(B, device="cuda"), tree["root_node"]].cpu().numpy()
        act = active.cpu().numpy()
        max_nc = int(nc.max()) if nc.size and nc.max() > 0 else 1
        noise = np.zeros((B, max_nc), dtype=np.float32)
        for i in range(B):
            n = int(nc[i])
            if n == 0 or not act[i]:
                continue
            alpha = max(0.03, min(cfg.dirichlet_alpha, 10.0 / n))
            noise[i, :n] = np.random.dirichlet([alpha] * n)
        self.ext.mcts_apply_root_noise(*self._tree_args(tree), torch.from_numpy(noise).cuda(), tree["root_node"],
                                       max_nc, cfg.dirichlet_epsilon, 1.0, B, self._max_nodes)

    def _run_simulations(self, tree, root_states, game_active, alive_mask, B, num_sims):  # :340-384
        cfg = self.config
        W = int(cfg.wave_size)
        leaf_states = torch.zeros((W * B, root_states.shape[1]), dtype=torch.uint8, device="cuda")
        for wave in range((num_sims + W - 1) // W):
            w = min(W, num_sims - wave * W)
            total = w * B
            leaf_idx, paths, plen, vl, vlen = self.ext.mcts_select_with_root_mask_batch(
                *self._tree_args(tree), tree["child_init_q"], game_active, tree["root_node"], alive_mask,
                self._max_legal, cfg.c_puct, B, w, self._max_nodes, False, 4.0, 0.0)
            leaves = leaf_states[:total]
            self.ext.mcts_replay_batch(root_states, leaves, paths[:total], plen[:total], leaf_idx[:total], B, total)
            results = self.ext.check_results_batch(leaves, total)
            legal, nl, feat = self.ext.generate_legal_moves_and_fnn_features_batch(leaves, total)
            priors, vals, child_q = self._eval_states(leaves, legal, nl, total, feat)
            self.ext.mcts_expand_and_backprop_dense_priors_batch(
                *self._tree_args(tree), tree["child_init_q"], child_q, leaf_idx[:total], leaves, legal, nl, priors,
                results, vals, vl[:total], vlen[:total], B, total, self._max_nodes, 0.0)

    def _gather_root_child_stats(self, tree, B):  # :388-410, vectorised
        row = torch.arange(B, device="cuda")
        root = tree["root_node"]
        fc = tree["first_child"][row, root].to(torch.int64)
        nc = tree["num_children"][row, root].to(torch.int64)
        lim = nc.clamp(max=self._max_legal)
        ok = (fc.unsqueeze(1) >= 0) & (self._slot_idx < lim.unsqueeze(1))
        idx = (fc.unsqueeze(1) + self._slot_idx).clamp(0, self._max_nodes - 1)
        r2 = row.unsqueeze(1).expand_as(idx)
        vc = torch.where(ok, tree["visit_count"][r2, idx], torch.zeros((), dtype=torch.int32, device="cuda"))
        tv = torch.where(ok, tree["total_value"][r2, idx], torch.zeros((), device="cuda"))
        q = torch.where(vc > 0, -tv / vc.clamp(min=1).float(), torch.zeros_like(tv))
        return vc, q

    def _reroot_tree(self, tree, B, moved, chosen_slot):  # :412-443
        fc = tree["first_child"][torch.arange(B, device="cuda"), tree["root_node"]]
        moved = moved & (fc >= 0)
        if self.config.rebase_tree_each_move:
            self._eval_helper._reset_games(tree, moved)
            return
        new_roots = torch.where(moved, (fc + chosen_slot.to(torch.int32)).to(torch.int32), tree["root_node"])
        tree["root_node"].copy_(new_roots)
        tree["parent_idx"].scatter_(1, new_roots.long().unsqueeze(1),
                                    torch.full((B, 1), -1, dtype=torch.int32, device="cuda"))

    # ---- one ply -------------------------------------------------------
    def search_ply(self, states, tree, active_mask, move_numbers):
        """Root evaluation + PUCT simulations + move choice for every active
        game (:160-239).  Returns (chosen_slot, legal, num_legal, policy,
        slot_visits, has_actions), or None when no game has a legal move."""
        cfg = self.config
        B = states.shape[0]
        # the fused leaf evaluation's head biases, read on the host once per ply
        self._eval_helper._head_biases = (float(self.net.value_fc.bias.item()),
                                          float(self.net.action_fc2.bias.item()))
        legal, nl, root_feat = self.ext.generate_legal_moves_and_fnn_features_batch(states, B)
        n64 = nl.to(torch.int64)
        has_actions = active_mask & (n64 > 0)
        wins = self._find_immediate_wins(states, legal, nl, B)
        has_win = wins >= 0
        if B == 0 or int(n64.max().item()) == 0:
            return None
        priors, _, child_q = self._eval_states(states, legal, nl, B, root_feat)
        any_win = bool(has_win.any().item())
        if any_win:
            priors.zero_()
            priors[has_win, wins[has_win]] = 1.0
            child_q.zero_()
        game_active = has_actions.to(torch.int8)
        self._expand_root_if_needed(tree, states, legal, nl, priors, child_q, game_active, B)
        self._apply_root_dirichlet(tree, B, has_actions)
        valid_slot = self._slot_idx < n64.unsqueeze(1)
        if any_win:
            slot_visits = torch.zeros(B, self._max_legal, dtype=torch.int32, device="cuda")
            slot_visits[has_win, wins[has_win]] = cfg.num_simulations
            probs = torch.zeros(B, self._max_legal, dtype=torch.float32, device="cuda")
            probs[has_win, wins[has_win]] = 1.0
        else:
            self._run_simulations(tree, states, game_active, valid_slot.to(torch.int8), B, cfg.num_simulations)
            slot_visits, _ = self._gather_root_child_stats(tree, B)
            vf = slot_visits.float()
            vsum = vf.sum(dim=1, keepdim=True)
            probs = torch.where(vsum > 0, vf / vsum.clamp(min=1.0), torch.zeros_like(vf))
            uniform = valid_slot.float()
            uniform = uniform / uniform.sum(dim=1, keepdim=True).clamp(min=1.0)
            probs = torch.where(vsum > 0, probs, uniform)
        chosen = torch.zeros((B,), dtype=torch.int64, device="cuda")
        active_idx = torch.nonzero(has_actions, as_tuple=False).squeeze(1)
        if any_win:
            chosen[has_win] = wins[has_win]
        elif active_idx.numel() > 0:
            greedy = move_numbers[active_idx] >= cfg.temperature_drop_move
            g_rows, s_rows = active_idx[greedy], active_idx[~greedy]
            if g_rows.numel() > 0:
                chosen[g_rows] = probs[g_rows].argmax(dim=1)
            if s_rows.numel() > 0:
                p = probs[s_rows]
                p = p / p.sum(dim=1, keepdim=True).clamp_min(1e-8)
                chosen[s_rows] = torch.multinomial(p, 1).squeeze(1)
        return chosen, legal, nl, probs, slot_visits, has_actions

    def self_play_batch(self, start_states: torch.Tensor | None = None) -> list[list[FNNTrainingExample]]:
        cfg = self.config
        B = cfg.batch_size
        states = start_states.cuda().contiguous() if start_states is not None else \
            self.ext.create_initial_states(B, cfg.expansion_mask)
        tree = self._alloc_tree(B)
        active = torch.ones((B,), dtype=torch.bool, device="cuda")
        move_numbers = torch.zeros((B,), dtype=torch.int64, device="cuda")
        histories: list[list] = [[] for _ in range(B)]
        while bool(active.any().item()):
            out = self.search_ply(states, tree, active, move_numbers)
            if out is None:
                break
            chosen, legal, nl, probs, _, has_actions = out
            active &= nl > 0
            has_cpu = has_actions.cpu().numpy()
            n_cpu = nl.cpu().numpy()
            st_cpu = states.cpu().numpy()
            pr_cpu = probs.cpu().numpy()
            for i in np.nonzero(has_cpu)[0]:
                histories[i].append((st_cpu[i].copy(), pr_cpu[i, : n_cpu[i]].astype(np.float32)))
            move = torch.zeros((B, 6), dtype=torch.uint8, device="cuda")
            idx = torch.nonzero(has_actions, as_tuple=False).squeeze(1)
            if idx.numel():
                move[idx] = legal[idx, chosen[idx].clamp(max=self._max_legal - 1)]
            self.ext.apply_moves_batch(states, move, B)
            self._reroot_tree(tree, B, has_actions, chosen)
            move_numbers += has_actions.to(torch.int64)
            res = self.ext.check_results_batch(states, B)
            active &= (res == 0) & (move_numbers < cfg.max_game_length)
        final = self.ext.check_results_batch(states, B).cpu().numpy()
        out_ex: list[list[FNNTrainingExample]] = [[] for _ in range(B)]
        for i in range(B):
            winner = int(final[i])
            use_v = winner != 0
            weighted_from = len(histories[i]) - max(0, int(cfg.final_value_ply_count))
            for h, (sb, pi) in enumerate(histories[i]):
                turn = int(sb[_OFF_TURN]) | (int(sb[_OFF_TURN + 1]) << 8)
                w = float(cfg.final_value_weight) if (use_v and h >= weighted_from) else 1.0
                out_ex[i].append(FNNTrainingExample(sb, pi.astype(np.float32),
                                                    float(FNNMCTSOrchestrator._result_to_value(winner, turn)),
                                                    True, use_v, w))
        return out_ex
