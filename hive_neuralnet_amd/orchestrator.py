"""Gumbel-root MCTS self-play over the MI355X engine: the counterpart of the
reference's FNNMCTSOrchestrator (hive_fnn/fnn_mcts_orchestrator.py).

Per ply (self_play_batch, :561-875): legal lists + root features, leaf
evaluation of every legal successor with the FNN (`_eval_states`,
:243-316), immediate-win override (:446-493), root candidates by prior with
queen-surround reserve slots (:384-444), root expansion (:888-902) and
Dirichlet noise (:904-925), four sequential-halving rounds of waves of
root-slot simulations (:670-711, :982-1055), final Gumbel argmax (:714-731),
visited-only policy target with adaptive temperature (:144-191, :738-755),
apply + rebase (:812-818, :1122-1142).

Differences from the reference, all deliberate:
  * ties in every top-k are broken by the lowest slot (a stable descending
    sort) -- torch.topk's tie order is unspecified, so the reference's is not
    reproducible;
  * per-game Python loops (immediate wins, tree rebase, history) are
    vectorised; the results are the same;
  * the tree kernels apply each game's simulations in simulation order (see
    include/hive_gpu.h), where the reference's atomics race.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

from . import hive_gpu
from .fnn import HiveFNN

_OFF_TURN = 3412
_OFF_HEIGHT = 2645
_OFF_QUEEN_CELL = 3392
_GUMBEL_ROUNDS = 4
_GUMBEL_WAVE_SCHEDULE = (2, 4, 8, 16)
_NUM_CELLS = 529


@dataclass
class FNNMCTSConfig:  # fnn_mcts_orchestrator.py:45-82 (same fields and defaults)
    num_simulations: int = 128
    max_num_considered_actions: int = 16
    c_puct: float = 1.25
    c_visit: float = 50.0
    c_scale: float = 1.0
    temperature: float = 1.0
    temperature_drop_move: int = 20
    batch_size: int = 128
    max_game_length: int = 300
    expansion_mask: int = 0
    wave_parallel: bool = True
    wave_size: int = 4
    deterministic_non_root: bool = False
    virtual_q_penalty: float = 0.25
    non_root_sigma: float = 4.0
    dirichlet_alpha: float = 0.3
    dirichlet_epsilon: float = 0.25
    max_tree_nodes: int = 65536
    queen_surround_reserve_slots: int = 6
    queen_surround_reserve_immobile_only: bool = True
    root_q_min_visits: int = 0
    short_forced_win_probe: bool = False
    probe_win_in_one: bool = True
    probe_check_opponent_wins: bool = True
    probe_win_in_two: bool = True
    policy_target_temperature: float = 1.0
    adaptive_policy_target_temperature: bool = True
    policy_target_top1_cap: float = 0.7
    policy_target_min_temperature: float = 1.0
    policy_target_max_temperature: float = 7.0
    final_value_ply_count: int = 3
    final_value_weight: float = 2.0
    rebase_tree_each_move: bool = True


@dataclass
class FNNTrainingExample:  # hive_fnn/fnn_replay_buffer.py:21-30 record shape
    state_bytes: np.ndarray
    policy_target: np.ndarray
    value_target: float
    use_for_policy: bool = True
    use_for_value: bool = True
    value_weight: float = 1.0
    surprise_weight: float = 1.0


@dataclass
class PlyResult:
    chosen_slot: torch.Tensor
    legal_moves: torch.Tensor
    num_legal: torch.Tensor
    policy: torch.Tensor
    slot_visits: torch.Tensor
    has_actions: torch.Tensor
    simulations: int = 0
    stats: dict = field(default_factory=dict)
    forced_random: torch.Tensor | None = None  # the root probe left no safe move: random move, no policy target


def topk_stable(x: torch.Tensor, k: int):
    """Top-k along dim 1, ties to the lowest index."""
    vals, idx = torch.sort(x, dim=1, descending=True, stable=True)
    return vals[:, :k], idx[:, :k]


# The streams of the game ranges, one set per device for the whole process:
# HIP maps streams onto a few hardware queues (4 by default), so streams made
# afresh by every orchestrator would end up sharing queues with each other and
# with the default stream, and the ranges would no longer overlap.
_RANGE_STREAMS: dict = {}


def _range_streams(parts: int) -> list:
    pool = _RANGE_STREAMS.setdefault(torch.cuda.current_device(), [])
    while len(pool) < parts:
        pool.append(torch.cuda.Stream())
    return pool


class FNNMCTSOrchestrator:
    def __init__(self, net: HiveFNN, config: FNNMCTSConfig | None = None) -> None:
        self.ext = hive_gpu.load_extension()
        self.config = config or FNNMCTSConfig()
        self.net = net
        self._max_nodes = int(self.config.max_tree_nodes)
        self._max_legal = int(self.ext.MAX_LEGAL_MOVES)
        self._slot_idx = torch.arange(self._max_legal, device="cuda", dtype=torch.int64).unsqueeze(0)
        self.last_policy_temperature_stats: dict[str, float] = {}
        # optional device-side counters (no host sync): simulations run, legal
        # moves at their leaves, virtual-loss path lengths, successor rows
        self.counters: dict[str, torch.Tensor] | None = None
        self.keep_last_leaves = False
        self.last_leaves: torch.Tensor | None = None
        # (value_fc.bias, action_fc2.bias) on the host, read once per search ply
        self._head_biases: tuple[float, float] | None = None
        # device workspace of the sync-free leaf evaluation (successor rows at
        # capacity 256 per leaf), kept across waves
        self._leaf_ws: torch.Tensor | None = None
        # simulation waves replayed from captured HIP graphs (one per wave shape):
        # True, False, or None = only waves of fewer than graph_rows rows, where
        # launch overhead is a large part of a wave (at 16 games x 1,024 sims,
        # 512-row waves, a ply runs 14% faster from graphs; with 2,048-row waves
        # it is even, and from 4,096 rows eager launches are faster, the graph's
        # input copies outweighing it)
        self.use_graphs: bool | None = None
        self.graph_rows = 2048
        self.max_graphs = 64
        self._graphs: dict = {}
        # the search phase of a ply -- every simulation wave of the four
        # rounds and the halving decisions, whose shapes the configuration
        # fixes -- replayed from one captured HIP graph: None = whenever every
        # round runs on one game range (and use_graphs is not False), True /
        # False = always / never.  The ply's candidates, Gumbel scores and
        # active games are copied into the graph's buffers before each replay.
        self.use_ply_graphs: bool | None = None
        self.max_ply_graphs = 4
        # game ranges of a captured ply, each range's waves a branch of the
        # graph (None = one).  At 512 games two branches measured no faster
        # with the wave schedule and 11 % slower with one simulation per
        # candidate per wave: the branches' kernels did not overlap.
        self.ply_graph_parts: int | None = None
        self._ply_graphs: dict = {}
        # simulation waves of disjoint game ranges on their own streams, so that
        # one range's latency-bound tree walks overlap another's leaf evaluation
        # (games are independent: results are identical to one range); None =
        # two ranges from split_min_games games and split_min_rows rows per
        # range and wave up (smaller waves are bound by host launches, which
        # ranges multiply), 1 = off
        self.game_parts: int | None = None
        self.split_min_games = 256
        self.split_min_rows = 8192
        self.max_game_parts = 1  # the most game ranges a simulation phase has used
        self._part_ws: dict = {}
        # simulation waves as one library call each (hg_mcts_wave_root_slots:
        # the tree, network and per-simulation buffers prepared once per buffer
        # set) wherever the fused leaf evaluation serves the network; False =
        # the step entry points one by one, in the reference's call sequence
        self.native_waves = True
        self._wave_plans: dict = {}
        # sequential-halving decisions (candidate statistics, sigma, scores,
        # survivors) as one kernel each (hg_gumbel_halving) for up to 64
        # considered actions; False = the torch ops
        self.native_halving = True
        self._packed: tuple | None = None

    def enable_counters(self) -> None:
        self._stats = torch.zeros((4,), dtype=torch.int64, device="cuda")
        self.counters = {k: self._stats[i] for i, k in enumerate(("sims", "leaf_legal", "vl_len", "rows"))}

    # ---- helpers -------------------------------------------------------
    def _rows(self, n: int) -> torch.Tensor:
        return torch.arange(n, device="cuda", dtype=torch.int64).unsqueeze(1)

    def _alloc_tree(self, B: int) -> dict:  # :195-214
        M = self._max_nodes
        z = lambda dt: torch.zeros(B, M, dtype=dt, device="cuda")  # noqa: E731
        return {
            "visit_count": z(torch.int32), "total_value": z(torch.float32), "prior": z(torch.float32),
            "virtual_q_penalty": z(torch.float32),
            "parent_idx": torch.full((B, M), -1, dtype=torch.int32, device="cuda"),
            "move_bytes": torch.zeros(B, M, 6, dtype=torch.uint8, device="cuda"),
            "action_idx": torch.full((B, M), -1, dtype=torch.int32, device="cuda"),
            "first_child": torch.full((B, M), -1, dtype=torch.int32, device="cuda"),
            "num_children": z(torch.int32), "is_terminal": z(torch.int8), "terminal_value": z(torch.float32),
            "node_count": torch.ones(B, dtype=torch.int32, device="cuda"),
            "root_node": torch.zeros(B, dtype=torch.int32, device="cuda"),
            "child_init_q": z(torch.float32),
        }

    def _reset_games(self, tree: dict, games: torch.Tensor) -> None:  # _reroot_tree rebase, :1122-1142
        """Hard rebase of the games flagged in `games` (bool [B])."""
        B = games.shape[0]
        self.ext.mcts_reset_trees(*self._tree_args(tree), tree["child_init_q"], games.contiguous(), tree["root_node"],
                                  B, self._max_nodes)

    def _tree_args(self, tree: dict) -> list:
        return [tree["visit_count"], tree["total_value"], tree["prior"], tree["parent_idx"],
                tree["virtual_q_penalty"], tree["move_bytes"], tree["action_idx"], tree["first_child"],
                tree["num_children"], tree["is_terminal"], tree["terminal_value"], tree["node_count"]]

    # ---- evaluation (:243-316) -----------------------------------------
    def _fused_eval_ok(self) -> bool:
        c = self.net.config
        return c.hidden_dim == 64 and c.embed_dim == 64 and c.action_hidden == 64

    def _eval_states(self, states, legal_moves, num_legal, total, root_features=None, workspace=None):
        """(priors [total, 256], leaf values [total], child Q [total, 256]).

        The 64-wide presets run the fused path, hg_fnn_leaf_eval_lists: the
        successor rows sized and mapped on the device (no host
        synchronisation per wave), their features written straight into the
        network input, then the whole network and the heads on matrix cores,
        softmax and the [T, 256] scatter.  Other widths run the torch
        composition of the reference (_eval_states_torch)."""
        if not self._fused_eval_ok():
            return self._eval_states_torch(states, legal_moves, num_legal, total, root_features)
        MAX_L = self._max_legal
        if root_features is None:
            root_features = self.ext.extract_fnn_features_batch(states, legal_moves, num_legal, total)
        if total == 0:
            empty = torch.zeros(0, MAX_L, dtype=torch.float32, device="cuda")
            return empty, empty.new_zeros((0,)), empty
        if workspace is None:
            need = self.ext.leaf_eval_workspace_bytes(total)
            if self._leaf_ws is None or self._leaf_ws.numel() < need:
                self._leaf_ws = torch.empty((need,), dtype=torch.uint8, device="cuda")
            workspace = self._leaf_ws
        return self.ext.fnn_leaf_eval_lists(states, legal_moves, num_legal, root_features.contiguous(), total,
                                            self.net, self._head_biases, workspace)

    def _eval_states_torch(self, states, legal_moves, num_legal, total, root_features=None):
        MAX_L = self._max_legal
        n64 = num_legal.to(torch.int64)
        if root_features is None:
            root_features = self.ext.extract_fnn_features_batch(states, legal_moves, num_legal, total)
        if total == 0:
            empty = torch.zeros(0, MAX_L, dtype=torch.float32, device="cuda")
            return empty, empty.new_zeros((0,)), empty
        valid = self._slot_idx < n64.unsqueeze(1)
        action_to_root = self._rows(total).expand_as(valid)[valid]
        move_indices = self._slot_idx.expand_as(valid)[valid]
        n_total = int(action_to_root.shape[0])
        if n_total == 0:
            with torch.inference_mode():
                root_values = self.net.value_head(self.net.encode(root_features)).squeeze(-1).float()
            z = torch.zeros(total, MAX_L, dtype=torch.float32, device="cuda")
            return z, root_values, z.clone()
        succ = self.ext.fnn_successor_features_batch(states, legal_moves, action_to_root, move_indices, n_total)
        with torch.inference_mode():
            emb = self.net.encode(torch.cat([root_features, succ], dim=0))
            root_emb, succ_emb = emb[:total], emb[total:]
            root_values = self.net.value_head(root_emb).squeeze(-1).float()
            child_values = self.net.value_head(succ_emb).squeeze(-1).float()
            logits = self.net.score_actions(root_emb[action_to_root], succ_emb).float()
        legal_logits = torch.full((total, MAX_L), -1e30, dtype=torch.float32, device="cuda")
        legal_logits[valid] = logits
        prior = torch.softmax(legal_logits, dim=1).masked_fill(~valid, 0.0)
        child_q = torch.zeros(total, MAX_L, dtype=torch.float32, device="cuda")
        child_q[valid] = -child_values
        return prior, root_values, child_q

    # ---- root candidates (:318-444) ------------------------------------
    def _queen_surround_qualifying_mask(self, states, legal_moves, num_legal, total):
        """Legal slots whose move raises the surround count of the opponent's
        queen (and, with queen_surround_reserve_immobile_only, leaves that side
        no queen escape): [total, 256] bool (hg_reserve_candidates)."""
        qual, _ = self.ext.reserve_candidates(states, legal_moves, num_legal, total,
                                              self.config.queen_surround_reserve_immobile_only)
        return qual

    def _root_candidate_slots(self, states, legal_moves, num_legal, priors, legal_logits, total,
                              allowed_slot_mask=None):  # :384-444
        max_legal = self._max_legal
        k = min(int(self.config.max_num_considered_actions), max_legal)
        valid = self._slot_idx < num_legal.to(torch.int64).unsqueeze(1)
        if allowed_slot_mask is not None:
            valid &= allowed_slot_mask
        reserve = min(int(self.config.queen_surround_reserve_slots), k)
        if reserve <= 0:
            u = torch.rand(total, max_legal, device="cuda").clamp(1e-4, 1 - 1e-4)
            g = torch.where(valid, -torch.log(-torch.log(u)), torch.full_like(u, -1e30))
            return topk_stable(g + legal_logits, k)[1].to(torch.int32)
        # qualification and the candidate row in one launch
        _, cand = self.ext.reserve_candidates(states, legal_moves, num_legal, total,
                                              self.config.queen_surround_reserve_immobile_only, priors=priors, k=k,
                                              reserve=reserve, allowed=allowed_slot_mask, want_qualifies=False)
        return cand

    def _candidate_row(self, qual, valid, priors, k, reserve):
        """The root candidate row (fnn_mcts_orchestrator.py:411-444) from a
        qualifying mask (hg_candidate_rows): `reserve` columns of qualifying
        slots by prior (-1 padded), then the other legal slots by prior, then
        the rest (reserved and illegal slots, lowest slot first), cut to k."""
        return self.ext.candidate_rows(qual, valid, priors, k, reserve)

    def _find_immediate_wins(self, states, legal_moves, num_legal, total):  # :446-493, vectorised
        winners = torch.full((total,), -1, dtype=torch.int64, device="cuda")
        valid = self._slot_idx < num_legal.to(torch.int64).unsqueeze(1)
        if total == 0 or not bool(valid.any().item()):
            return winners
        a2r = self._rows(total).expand_as(valid)[valid]
        mi = self._slot_idx.expand_as(valid)[valid]
        n_total = int(a2r.shape[0])
        child = states[a2r].clone()
        self.ext.apply_moves_batch(child, legal_moves[a2r, mi].contiguous(), n_total)
        results = self.ext.check_results_batch(child, n_total)
        is_white = (states[a2r, _OFF_TURN].to(torch.int32) % 2) == 0
        win = ((results == 1) & is_white) | ((results == 2) & ~is_white)
        first = torch.full((total,), self._max_legal, dtype=torch.int64, device="cuda")
        first.scatter_reduce_(0, a2r[win], mi[win], reduce="amin")
        return torch.where(first < self._max_legal, first, winners)

    # ---- tree steps ----------------------------------------------------
    def _expand_root_if_needed(self, tree, states, legal_moves, num_legal, priors, child_q, game_active, B):
        root = tree["root_node"]
        fc = tree["first_child"][torch.arange(B, device="cuda"), root]
        needs = (fc < 0) & game_active.to(torch.bool)
        if not bool(needs.any().item()):
            return
        leaf = torch.where(needs, root.to(torch.int32), torch.full_like(root, -1, dtype=torch.int32))
        results = self.ext.check_results_batch(states, B)
        self.ext.mcts_expand_dense_priors_batch(*self._tree_args(tree), tree["child_init_q"], child_q, leaf, states,
                                                legal_moves, num_legal, priors, results, B, B, self._max_nodes)

    def _apply_root_dirichlet(self, tree, B, active):  # :904-925
        cfg = self.config
        nc = tree["num_children"][torch.arange(B, device="cuda"), tree["root_node"]].cpu().numpy()
        act = active.cpu().numpy()
        max_nc = int(nc.max()) if nc.size and nc.max() > 0 else 1
        noise = np.zeros((B, max_nc), dtype=np.float32)
        # Dirichlet(alpha_g, ..., alpha_g) for every active game at once: independent
        # Gamma(alpha_g) draws normalised per game (the same law as one
        # np.random.dirichlet call per game); a game whose draws all underflow
        # to 0 takes np.random.dirichlet itself
        games = np.nonzero((nc > 0) & act)[0]
        if games.size:
            n = nc[games].astype(np.int64)
            alpha = np.maximum(0.03, np.minimum(cfg.dirichlet_alpha, 10.0 / n))
            draws = np.random.standard_gamma(np.repeat(alpha, n))
            starts = np.concatenate([[0], np.cumsum(n)[:-1]])
            sums = np.add.reduceat(draws, starts)
            cols = np.arange(int(n.sum())) - np.repeat(starts, n)
            rows = np.repeat(games, n)
            ok = np.repeat(sums > 0, n)
            noise[rows[ok], cols[ok]] = (draws / np.repeat(np.where(sums > 0, sums, 1.0), n))[ok]
            for k in np.nonzero(sums <= 0)[0]:
                noise[games[k], : n[k]] = np.random.dirichlet([alpha[k]] * int(n[k]))
        self.ext.mcts_apply_root_noise(*self._tree_args(tree), torch.from_numpy(noise).cuda(), tree["root_node"],
                                       max_nc, cfg.dirichlet_epsilon, 1.0, B, self._max_nodes)

    def _game_parts_for(self, B, C, W):
        """Game ranges of a round's waves (W simulations per candidate column, C columns)."""
        if self.game_parts is not None:
            return self.game_parts
        return 2 if B >= self.split_min_games and W * C * B >= 2 * self.split_min_rows else 1

    def _run_simulations_for_root_slots(self, tree, root_states, game_active, root_slots, B, per_slot, wave_size):
        cfg = self.config
        C = int(root_slots.shape[1])
        W = max(1, int(wave_size))
        q_penalty = float(cfg.virtual_q_penalty) if cfg.deterministic_non_root and W > 1 else 0.0
        parts = self._game_parts_for(B, C, W)
        if parts > 1 and B >= parts:
            self.max_game_parts = max(self.max_game_parts, parts)
            return self._run_split(tree, root_states, game_active, root_slots, B, C, per_slot, W, q_penalty, parts)
        sims = 0
        for wave in range(math.ceil(per_slot / W)):
            w = min(W, per_slot - wave * W)
            total = w * C * B
            graphs = self.use_graphs if self.use_graphs is not None else total < self.graph_rows
            if graphs:
                leaf_idx, leaf_states, nl, vlen = self._graph_wave(tree, root_states, game_active, root_slots, C, B,
                                                                  w, q_penalty)
                if self.counters is not None:
                    self.ext.mcts_wave_stats(leaf_idx, nl, vlen, total, self._stats)
            else:
                leaf_idx, leaf_states, nl, vlen = self._wave(tree, root_states, game_active, root_slots, C, B, w,
                                                             q_penalty)
            if self.keep_last_leaves:
                self.last_leaves = leaf_states[leaf_idx >= 0]
            sims += total
        return sims

    def _run_split(self, tree, root_states, game_active, root_slots, B, C, per_slot, W, q_penalty, parts):
        """The waves of _run_simulations_for_root_slots over `parts` contiguous
        game ranges, each range's waves in order on its own stream (default
        priority), the ranges' launches interleaved wave by wave.  Every tree
        array is per game ([B, ...] rows), so a range is a set of row views;
        the ranges share nothing but the device-atomic wave counters."""
        bounds = [(B * p) // parts for p in range(parts + 1)]
        streams = _range_streams(parts)
        main = torch.cuda.current_stream()
        ready = torch.cuda.Event()
        ready.record(main)
        ranges = []
        for p in range(parts):
            lo, hi = bounds[p], bounds[p + 1]
            s = streams[p]
            s.wait_event(ready)
            ranges.append((p, {k: v[lo:hi] for k, v in tree.items()}, root_states[lo:hi], game_active[lo:hi],
                           root_slots[lo:hi], hi - lo, s))
        sims = 0
        waves = math.ceil(per_slot / W)
        last = []
        for wave in range(waves):
            w = min(W, per_slot - wave * W)
            for p, tv, rs, ga, sl, nb, s in ranges:
                with torch.cuda.stream(s):
                    total = w * C * nb
                    if self._native_waves_ok():
                        leaf_idx, leaf_states, nl, vlen = self._wave(
                            tv, rs, ga, sl, C, nb, w, q_penalty, plan=self._wave_plan(("part", p), tv, nb, total))
                    else:
                        need = self.ext.leaf_eval_workspace_bytes(total)
                        ws = self._part_ws.get(p)
                        if ws is None or ws.numel() < need:
                            ws = torch.empty((need,), dtype=torch.uint8, device="cuda")
                            self._part_ws[p] = ws
                        leaf_idx, leaf_states, nl, vlen = self._wave(tv, rs, ga, sl, C, nb, w, q_penalty, ws)
                    if self.keep_last_leaves and wave == waves - 1:
                        last.append(leaf_states[leaf_idx >= 0])
            sims += w * C * B
        for r in ranges:
            done = torch.cuda.Event()
            done.record(r[-1])
            main.wait_event(done)
        if last:
            self.last_leaves = torch.cat(last)
        return sims

    def _packed_tree(self, tree, B):
        """The tree's arrays packed as an `hg_tree` (kept while they stay put)."""
        key = (tuple(v.data_ptr() for v in tree.values()), B)
        if self._packed is None or self._packed[0] != key:
            self._packed = (key, self.ext.tree_struct(*self._tree_args(tree), tree["child_init_q"], B,
                                                      self._max_nodes))
        return self._packed[1]

    def _native_waves_ok(self) -> bool:
        return self.native_waves and self._fused_eval_ok()

    def _wave_plan(self, slot, tree, B, total):
        """The WavePlan of buffer set `slot`: re-made for another tree or B or
        when a wave outgrows its buffers, re-pointed when the network (its
        parameter addresses or head biases) changes."""
        key = (tuple(v.data_ptr() for v in tree.values()), B)
        net_key = tuple(p.data_ptr() for p in self.net.parameters()) + tuple(self._head_biases or ())
        entry = self._wave_plans.get(slot)
        if entry is None or entry[0] != key or entry[1].capacity < total:
            self._wave_plans.pop(slot, None)  # release the old buffers first
            plan = self.ext.prepare_wave_root_slots(*self._tree_args(tree), tree["child_init_q"], B, self._max_nodes,
                                                    self.net, self._head_biases, capacity=total)
            entry = [key, plan, net_key]
            self._wave_plans[slot] = entry
        elif entry[2] != net_key:
            entry[1].set_net(self.net, self._head_biases)
            entry[2] = net_key
        return entry[1]

    def _wave(self, tree, root_states, game_active, root_slots, C, B, w, q_penalty, workspace=None, plan=None,
              stats=True):
        """One wave of w simulations per root candidate (:982-1055): select ->
        replay -> legal + features -> leaf evaluation -> expansion + backup,
        and the search counters when enabled and `stats`.  No host
        synchronisation.  Native waves (one library call) run on `plan`, or
        on the single-range buffer set.  Returns (leaf_idx, leaf_states,
        num_legal, vl_lens)."""
        cfg = self.config
        total = w * C * B
        counters = self._stats if (stats and self.counters is not None) else None
        if self._native_waves_ok():
            if plan is None:
                plan = self._wave_plan("main", tree, B, total)
            return plan.run(root_states, game_active, tree["root_node"], root_slots, C, self._max_legal, cfg.c_puct,
                            w, cfg.deterministic_non_root, cfg.non_root_sigma, q_penalty, stats=counters)
        (leaf_idx, leaf_states, legal, nl, feat, results, vl, vlen) = \
            self.ext.mcts_select_replay_legal_fnn_root_slots_batch(
                *self._tree_args(tree), tree["child_init_q"], root_states, game_active, tree["root_node"],
                root_slots, C, self._max_legal, cfg.c_puct, B, w, self._max_nodes, cfg.deterministic_non_root,
                cfg.non_root_sigma, q_penalty)
        priors, vals, child_q = self._eval_states(leaf_states, legal, nl, total, feat, workspace)
        self.ext.mcts_expand_and_backprop_dense_priors_batch(
            *self._tree_args(tree), tree["child_init_q"], child_q, leaf_idx, leaf_states, legal, nl, priors,
            results, vals, vl, vlen, B, total, self._max_nodes, q_penalty)
        if counters is not None:
            self.ext.mcts_wave_stats(leaf_idx, nl, vlen, total, counters)
        return leaf_idx, leaf_states, nl, vlen

    def _graph_wave(self, tree, root_states, game_active, root_slots, C, B, w, q_penalty):
        """_wave replayed from a captured HIP graph.  A graph is kept per wave
        shape, tree and root-state tensor; the active games and root slots are
        copied into the graph's own buffers before each replay, the root states
        and the network enter by address (parameter addresses and head biases
        are part of the key).  The graph holds only kernel launches (the extension fills
        and zeroes with kernels, never memset nodes)."""
        cfg = self.config
        net_key = tuple(p.data_ptr() for p in self.net.parameters()) + tuple(self._head_biases or ())
        tree_key = tuple(v.data_ptr() for v in tree.values())
        key = (tree_key, B, C, w, float(q_penalty), bool(cfg.deterministic_non_root), float(cfg.c_puct),
               float(cfg.non_root_sigma), root_states.data_ptr(), tuple(root_states.shape), net_key)
        entry = self._graphs.get(key)
        if entry is None:
            if len(self._graphs) >= self.max_graphs:  # oldest first
                self._graphs.pop(next(iter(self._graphs)))
            # the root states enter by address (part of the key: a ply's states
            # do not move); the per-round inputs are copied into the graph's buffers
            static = {"roots": root_states, "active": game_active.clone(), "slots": root_slots.clone()}
            # the graph's own buffers (a wave plan, or the leaf-evaluation workspace
            # of the step entry points), allocated outside capture and kept alive
            # with the graph; its counters are added after each replay
            if self._native_waves_ok():
                ws = self.ext.prepare_wave_root_slots(*self._tree_args(tree), tree["child_init_q"], B,
                                                      self._max_nodes, self.net, self._head_biases,
                                                      capacity=w * C * B)
                wave = dict(plan=ws)
            else:
                ws = torch.empty((self.ext.leaf_eval_workspace_bytes(w * C * B),), dtype=torch.uint8, device="cuda")
                wave = dict(workspace=ws)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                outs = self._wave(tree, static["roots"], static["active"], static["slots"], C, B, w, q_penalty,
                                  stats=False, **wave)
            entry = (graph, static, outs, ws)
            self._graphs[key] = entry
            # capture records the launches without running them: the replay below runs this wave
        graph, static, outs, _ = entry
        static["active"].copy_(game_active)
        static["slots"].copy_(root_slots)
        graph.replay()
        return outs

    def _round_shapes(self, C):
        """(C, per_slot, W) of each of the four rounds for C candidate columns."""
        cfg = self.config
        per_round = max(1, cfg.num_simulations // _GUMBEL_ROUNDS)
        out = []
        for r in range(_GUMBEL_ROUNDS):
            W = _GUMBEL_WAVE_SCHEDULE[min(r, len(_GUMBEL_WAVE_SCHEDULE) - 1)] if cfg.wave_parallel else 1
            out.append((C, max(1, per_round // C), W))
            if C > 1:
                C //= 2
        return out

    def _ply_graph_ok(self, B, C) -> bool:
        if self.use_ply_graphs is False or self.use_graphs is False or self.keep_last_leaves:
            return False
        if not (self._native_waves_ok() and self.native_halving and C <= 64):
            return False
        if self.ply_graph_parts is not None or self.use_ply_graphs:
            return True
        # by default only where every round's waves run on one game range
        return all(self._game_parts_for(B, c, w) <= 1 or B < self._game_parts_for(B, c, w)
                   for c, _, w in self._round_shapes(C))

    def _ply_graph_parts(self, B) -> int:
        """Game ranges of a captured ply (ply_graph_parts, default 1): each
        range's waves are a branch of the graph of their own."""
        return max(1, min(int(self.ply_graph_parts or 1), B))

    def _ply_graph(self, tree, root_states, game_active, cand, base, B):
        """_sequential_halving (fnn_mcts_orchestrator.py:650-731) replayed from a
        captured HIP graph: every wave of the four rounds on one buffer set of its
        own (hg_mcts_wave_root_slots), the halving decisions (hg_gumbel_halving)
        and the final choice.  Kept per tree, root-state tensor, network, counters
        and search configuration; the candidates, Gumbel scores and active games
        are copied into the graph's buffers before each replay.  Holds only
        kernel launches (no memset nodes).  Returns (chosen slot [B] int64,
        simulations)."""
        cfg = self.config
        C = int(cand.shape[1])
        parts = self._ply_graph_parts(B)
        net_key = tuple(p.data_ptr() for p in self.net.parameters()) + tuple(self._head_biases or ())
        stats = self._stats if self.counters is not None else None
        key = (tuple(v.data_ptr() for v in tree.values()), B, C, parts, root_states.data_ptr(), net_key,
               stats.data_ptr() if stats is not None else None, cfg.num_simulations, bool(cfg.wave_parallel),
               float(cfg.c_puct), bool(cfg.deterministic_non_root), float(cfg.non_root_sigma),
               float(cfg.virtual_q_penalty), float(cfg.c_visit), float(cfg.c_scale), int(cfg.root_q_min_visits))
        entry = self._ply_graphs.get(key)
        if entry is None:
            if len(self._ply_graphs) >= self.max_ply_graphs:  # oldest first
                self._ply_graphs.pop(next(iter(self._ply_graphs)))
            static = {"cand": cand.clone(), "base": base.clone(), "active": game_active.clone()}
            # one buffer set per game range; the ranges' waves are branches of the
            # graph (forked from the capture stream per round, joined before the
            # round's halving decision, which reads every game)
            bounds = [(B * p) // parts for p in range(parts + 1)]
            ranges = []
            for p in range(parts):
                lo, hi = bounds[p], bounds[p + 1]
                tv = {k: v[lo:hi] for k, v in tree.items()}
                cap = max(min(w, per) * c * (hi - lo) for c, per, w in self._round_shapes(C))
                plan = self.ext.prepare_wave_root_slots(*self._tree_args(tv), tv["child_init_q"], hi - lo,
                                                        self._max_nodes, self.net, self._head_biases, capacity=cap)
                ranges.append((lo, hi, plan, root_states[lo:hi], static["active"][lo:hi], tv["root_node"]))
            side = _range_streams(parts)
            hg_tree = self._packed_tree(tree, B)

            def run_round(c, per_slot, wave):
                W = max(1, int(wave))
                q_penalty = float(cfg.virtual_q_penalty) if cfg.deterministic_non_root and W > 1 else 0.0
                Cc = int(c.shape[1])
                main = torch.cuda.current_stream()
                if parts > 1:
                    fork = torch.cuda.Event()
                    fork.record(main)
                    for p in range(1, parts):
                        side[p].wait_event(fork)
                sims = 0
                for k in range(math.ceil(per_slot / W)):
                    w = min(W, per_slot - k * W)
                    for p, (lo, hi, plan, rs, act, rn) in enumerate(ranges):
                        with torch.cuda.stream(main if p == 0 else side[p]):
                            plan.run(rs, act, rn, c[lo:hi], Cc, self._max_legal, cfg.c_puct, w,
                                     cfg.deterministic_non_root, cfg.non_root_sigma, q_penalty, stats=stats)
                    sims += w * Cc * B
                for p in range(1, parts):
                    join = torch.cuda.Event()
                    join.record(side[p])
                    main.wait_event(join)
                return sims

            def decide(c, final):
                return self.ext.gumbel_halving(hg_tree, tree["root_node"], c, static["base"], cfg.c_visit,
                                               cfg.c_scale, int(cfg.root_q_min_visits), final)

            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                chosen, sims = self._sequential_halving(static["cand"], static["base"], run_round, None, decide)
            entry = (graph, static, chosen, sims, ranges, hg_tree)
            self._ply_graphs[key] = entry
            # capture records the launches without running them: the replay below runs this ply
        graph, static, chosen, sims = entry[:4]
        static["cand"].copy_(cand)
        static["base"].copy_(base)
        static["active"].copy_(game_active)
        graph.replay()
        return chosen.clone(), sims

    def _root_child_stats(self, tree, B, slots):  # _gather_root_candidate_stats / _gather_root_child_stats
        row = torch.arange(B, device="cuda", dtype=torch.long)
        root = tree["root_node"]
        fc = tree["first_child"][row, root].to(torch.long)
        nc = tree["num_children"][row, root].to(torch.long)
        slots = slots.to(torch.long)
        valid = (slots >= 0) & (fc.unsqueeze(1) >= 0) & (slots < nc.unsqueeze(1))
        idx = (fc.unsqueeze(1) + slots.clamp(min=0)).clamp(0, self._max_nodes - 1)
        r2 = row.unsqueeze(1).expand_as(idx)
        v_raw = tree["visit_count"][r2, idx]
        t_raw = tree["total_value"][r2, idx]
        visits = torch.where(valid, v_raw, torch.zeros_like(v_raw))
        q = torch.where(valid & (v_raw > int(self.config.root_q_min_visits)),
                        -t_raw / v_raw.clamp(min=1).float(), torch.zeros_like(t_raw))
        return visits, q

    def _build_policy_target(self, sampled_logits, valid_slot):  # :144-191
        cfg = self.config

        def soft(temp):
            p = torch.softmax(sampled_logits / temp, dim=1)
            p = torch.where(valid_slot, p, torch.zeros_like(p))
            return p / p.sum(dim=1, keepdim=True).clamp_min(1e-12)

        if not cfg.adaptive_policy_target_temperature:
            t = torch.full((sampled_logits.shape[0], 1), max(float(cfg.policy_target_temperature), 1e-6),
                           dtype=sampled_logits.dtype, device=sampled_logits.device)
            return soft(t), t.squeeze(1)
        lo_t = max(float(cfg.policy_target_min_temperature), 1.0)
        hi_t = max(float(cfg.policy_target_max_temperature), lo_t)
        cap = min(max(float(cfg.policy_target_top1_cap), 0.0), 1.0)
        base = torch.full((sampled_logits.shape[0], 1), lo_t, dtype=sampled_logits.dtype,
                          device=sampled_logits.device)
        probs = soft(base)
        need = probs.max(dim=1, keepdim=True).values > cap
        if not bool(need.any().item()) or hi_t <= lo_t:
            return probs, base.squeeze(1)
        low, high = base.clone(), torch.full_like(base, hi_t)
        for _ in range(12):
            mid = (low + high) * 0.5
            sharp = soft(mid).max(dim=1, keepdim=True).values > cap
            low = torch.where(need & sharp, mid, low)
            high = torch.where(need & ~sharp, mid, high)
        final = torch.where(need, high, base)
        return soft(final), final.squeeze(1)

    # ---- one ply of search ---------------------------------------------
    def search_ply(self, states: torch.Tensor, tree: dict, active_mask: torch.Tensor) -> PlyResult:
        """Root evaluation + Gumbel sequential halving for every active game (:589-755)."""
        cfg = self.config
        cfg.max_num_considered_actions = max(1, min(cfg.max_num_considered_actions, self._max_legal))
        B = states.shape[0]
        MAX_L = self._max_legal
        legal, nl, root_feat = self.ext.generate_legal_moves_and_fnn_features_batch(states, B)
        self._head_biases = (float(self.net.value_fc.bias.item()), float(self.net.action_fc2.bias.item()))
        n64 = nl.to(torch.int64)
        has_actions = active_mask & (n64 > 0)
        priors, _, child_q = self._eval_states(states, legal, nl, B, root_feat)
        valid_slot = self._slot_idx < n64.unsqueeze(1)
        allowed = valid_slot
        forced = torch.zeros((B,), dtype=torch.bool, device="cuda")
        if cfg.short_forced_win_probe:  # _analyze_short_tactics, :527-545 / :611-617
            wins, allowed_u8, forced_u8 = self.ext.root_tactical_probe_batch(
                states, legal, nl, priors, B, cfg.probe_win_in_one, cfg.probe_check_opponent_wins,
                cfg.probe_win_in_two)
            allowed = allowed_u8.to(torch.bool) & valid_slot
            forced = forced_u8.to(torch.bool) & has_actions
        else:
            wins = self._find_immediate_wins(states, legal, nl, B)
        has_win = wins >= 0
        if bool(has_win.any().item()):
            # the reference clears priors and child Q of EVERY game in the batch
            # once any game has a winning move (fnn_mcts_orchestrator.py:624-627)
            priors.zero_()
            priors[has_win, wins[has_win]] = 1.0
            child_q.zero_()
        search_rows = has_actions & ~has_win & ~forced
        legal_logits = torch.where(allowed, priors.clamp(min=1e-20).log(), torch.full_like(priors, -1e30))
        u = torch.rand(B, MAX_L, device="cuda").clamp(1e-4, 1 - 1e-4)
        gumbel = torch.where(allowed, -torch.log(-torch.log(u)), torch.full_like(u, -1e30))
        topk_slots = self._root_candidate_slots(states, legal, nl, priors, legal_logits, B, allowed)
        game_active = search_rows.to(torch.int8)
        self._expand_root_if_needed(tree, states, legal, nl, priors, child_q, game_active, B)
        self._apply_root_dirichlet(tree, B, search_rows)
        slot_visits = torch.zeros(B, MAX_L, dtype=torch.int32, device="cuda")
        probs = torch.zeros(B, MAX_L, dtype=torch.float32, device="cuda")
        chosen = torch.zeros((B,), dtype=torch.long, device="cuda")
        sims = 0
        stats: dict = {}
        if bool(search_rows.any().item()):
            cand = topk_slots.to(torch.int32)
            cvalid = torch.gather(valid_slot, 1, cand.long().clamp(min=0)) & (cand >= 0)
            cand = torch.where(cvalid, cand, torch.full_like(cand, -1))
            base = gumbel + legal_logits
            decide = None
            if self.native_halving and cand.shape[1] <= 64:
                hg_tree = self._packed_tree(tree, B)
                decide = lambda c, final: self.ext.gumbel_halving(  # noqa: E731
                    hg_tree, tree["root_node"], c, base, cfg.c_visit, cfg.c_scale, int(cfg.root_q_min_visits), final)
            if self._ply_graph_ok(B, int(cand.shape[1])):
                chosen, sims = self._ply_graph(tree, states, game_active, cand, base, B)
            else:
                chosen, sims = self._sequential_halving(
                    cand, base,
                    lambda c, per_slot, wave: self._run_simulations_for_root_slots(tree, states, game_active, c, B,
                                                                                   per_slot, wave),
                    lambda c: self._root_child_stats(tree, B, c), decide)
            slot_visits, slot_q = self._root_child_stats(tree, B, self._slot_idx.expand(B, -1))
            visited = (slot_visits > 0) & valid_slot
            max_n = slot_visits.float().max(dim=1, keepdim=True).values
            sampled = torch.where(visited, legal_logits + (cfg.c_visit + max_n) * cfg.c_scale * slot_q,
                                  torch.full_like(legal_logits, -1e30))
            probs, temps = self._build_policy_target(sampled, valid_slot)
            used = search_rows & visited.any(dim=1)
            if bool(used.any().item()):
                t = temps[used].detach().float().cpu().numpy()
                stats = {"sum": float(t.sum()), "count": int(t.shape[0]), "min": float(t.min()),
                         "max": float(t.max())}
        if bool(has_win.any().item()):
            slot_visits[has_win] = 0
            slot_visits[has_win, wins[has_win]] = cfg.num_simulations
            probs[has_win] = 0.0
            probs[has_win, wins[has_win]] = 1.0
            chosen = torch.where(has_win, wins, chosen)
        if bool(forced.any().item()):  # no safe move: a uniform random one, no policy target (:768-776)
            rand_slots = (torch.rand((B,), device="cuda") * n64.clamp(min=1).to(torch.float32)).to(torch.int64)
            chosen = torch.where(forced, rand_slots, chosen)
            probs = torch.where(forced.unsqueeze(1), torch.zeros_like(probs), probs)
        return PlyResult(chosen, legal, nl, probs, slot_visits, has_actions, sims, stats, forced)

    def _sequential_halving(self, cand, base, run_round, child_stats, decide=None):
        """Gumbel sequential halving (fnn_mcts_orchestrator.py:650-731).

        cand [B, C] int32 root slots (-1 = none); base [B, 256] = Gumbel noise +
        legal logits.  Round r (of 4) calls run_round(cand, per_slot, wave): per_slot
        = max(1, (simulations // 4) // C) simulations per candidate column, in waves
        of `wave` per column ((2, 4, 8, 16)[r], or 1 without wave_parallel); unless
        C = 1 it then keeps, in C // 2 columns, the top max(1, valid // 2)
        candidates by base[slot] + sigma * q, where (visits, q) = child_stats(cand)
        and sigma = (c_visit + the largest visit count of any candidate in the
        batch) * c_scale.  The final choice is the argmax of the same score over
        the survivors.  `decide(cand, final)`, when given, makes each of these
        decisions in one call (hg_gumbel_halving) instead of the torch ops:
        the next round's candidates, or with `final` the chosen slot.
        Returns (chosen slot [B] int64, simulations run)."""
        cfg = self.config
        B = cand.shape[0]
        sims = 0
        per_round = max(1, cfg.num_simulations // _GUMBEL_ROUNDS)
        for r in range(_GUMBEL_ROUNDS):
            cvalid = cand >= 0
            C = int(cand.shape[1])
            wave = _GUMBEL_WAVE_SCHEDULE[min(r, len(_GUMBEL_WAVE_SCHEDULE) - 1)] if cfg.wave_parallel else 1
            sims += run_round(cand, max(1, per_round // C), wave)
            if C <= 1:
                continue
            if decide is not None:
                cand = decide(cand, False)
                continue
            keep_n = (cvalid.sum(dim=1) // 2).clamp(min=1)
            max_keep = C // 2
            visits, q = child_stats(cand)
            sigma = (cfg.c_visit + visits.max()) * cfg.c_scale
            score = (torch.gather(base, 1, cand.long().clamp(min=0)) + sigma * q).float()
            score = torch.where(cvalid, score, torch.full_like(score, -1e30))
            _, keep_pos = topk_stable(score, max_keep)
            keep_ok = torch.arange(max_keep, device="cuda").unsqueeze(0) < keep_n.unsqueeze(1)
            cand = torch.where(keep_ok, torch.gather(cand, 1, keep_pos), torch.full_like(keep_pos, -1,
                                                                                        dtype=torch.int32))
        if decide is not None:
            return decide(cand, True), sims
        cvalid = cand >= 0
        visits, q = child_stats(cand)
        sigma = (cfg.c_visit + visits.max()) * cfg.c_scale
        final = (torch.gather(base, 1, cand.long().clamp(min=0)) + sigma * q).float()
        final = torch.where(cvalid, final, torch.full_like(final, -1e30))
        pos = torch.argmax(final, dim=1)
        chosen = torch.gather(cand, 1, pos.unsqueeze(1)).squeeze(1).clamp(min=0).to(torch.long)
        return chosen, sims

    def apply_and_rebase(self, states, tree, ply: PlyResult):
        B = states.shape[0]
        move = torch.zeros((B, 6), dtype=torch.uint8, device="cuda")
        idx = torch.nonzero(ply.has_actions, as_tuple=False).squeeze(1)
        if idx.numel():
            move[idx] = ply.legal_moves[idx, ply.chosen_slot[idx].clamp(max=self._max_legal - 1)]
        self.ext.apply_moves_batch(states, move, B)
        fc = tree["first_child"][torch.arange(B, device="cuda"), tree["root_node"]]
        moved = ply.has_actions & (fc >= 0)
        if self.config.rebase_tree_each_move:
            self._reset_games(tree, moved)
            return
        # keep the chosen child's subtree (fnn_mcts_orchestrator.py:1143-1153)
        new_roots = torch.where(moved, (fc + ply.chosen_slot.to(torch.int32)).to(torch.int32), tree["root_node"])
        tree["root_node"].copy_(new_roots)
        tree["parent_idx"].scatter_(1, new_roots.long().unsqueeze(1),
                                    torch.full((B, 1), -1, dtype=torch.int32, device="cuda"))

    # ---- full games ----------------------------------------------------
    def self_play_batch(self, start_states: torch.Tensor | None = None) -> list[list[FNNTrainingExample]]:
        cfg = self.config
        B = cfg.batch_size
        states = start_states.cuda().contiguous() if start_states is not None else \
            self.ext.create_initial_states(B, cfg.expansion_mask)
        tree = self._alloc_tree(B)
        active = torch.ones((B,), dtype=torch.bool, device="cuda")
        moves_done = torch.zeros((B,), dtype=torch.int64, device="cuda")
        histories: list[list] = [[] for _ in range(B)]
        t_sum, t_count, t_min, t_max = 0.0, 0, float("inf"), 0.0
        while bool(active.any().item()):
            ply = self.search_ply(states, tree, active)
            if ply.stats:
                t_sum += ply.stats["sum"]
                t_count += ply.stats["count"]
                t_min = min(t_min, ply.stats["min"])
                t_max = max(t_max, ply.stats["max"])
            active &= ply.num_legal > 0
            if not bool(ply.has_actions.any().item()):
                break
            has_cpu = ply.has_actions.cpu().numpy()
            n_cpu = ply.num_legal.cpu().numpy()
            st_cpu = states.cpu().numpy()
            pr_cpu = ply.policy.cpu().numpy()
            fr_cpu = ply.forced_random.cpu().numpy() if ply.forced_random is not None else np.zeros_like(has_cpu)
            for i in np.nonzero(has_cpu)[0]:
                histories[i].append((st_cpu[i].copy(), pr_cpu[i, : n_cpu[i]].astype(np.float32), not fr_cpu[i]))
            self.apply_and_rebase(states, tree, ply)
            moves_done += ply.has_actions.to(torch.int64)
            res = self.ext.check_results_batch(states, B)
            active &= (res == 0) & (moves_done < cfg.max_game_length)
        final = self.ext.check_results_batch(states, B).cpu().numpy()
        out: list[list[FNNTrainingExample]] = [[] for _ in range(B)]
        for i in range(B):
            winner = int(final[i])
            use_v = winner != 0
            weighted_from = len(histories[i]) - max(0, int(cfg.final_value_ply_count))
            for h, (sb, pi, use_p) in enumerate(histories[i]):
                turn = int(sb[_OFF_TURN]) | (int(sb[_OFF_TURN + 1]) << 8)
                value = self._result_to_value(winner, turn)
                w = float(cfg.final_value_weight) if (use_v and h >= weighted_from) else 1.0
                out[i].append(FNNTrainingExample(sb, pi, float(value), use_p, use_v, w))
        if t_count:
            self.last_policy_temperature_stats = {"mean": t_sum / t_count, "min": t_min, "max": t_max,
                                                  "count": float(t_count)}
        else:
            lo = float(cfg.policy_target_min_temperature)
            self.last_policy_temperature_stats = {"mean": lo, "min": lo, "max": lo, "count": 0.0}
        return out

    @staticmethod
    def _result_to_value(result: int, turn: int) -> float:  # :1155-1161
        if result == 0 or result == 3:
            return 0.0
        white = turn % 2 == 0
        return 1.0 if (result == 1 and white) or (result == 2 and not white) else -1.0
