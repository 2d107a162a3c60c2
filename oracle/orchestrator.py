"""Numpy restatement of one Gumbel search ply of the self-play orchestrator.

TEST INFRASTRUCTURE ONLY.  It follows hive_fnn/fnn_mcts_orchestrator.py
(self_play_batch :589-766 and the helpers :144-191, :318-493, :879-1120)
step by step with numpy and the C oracles (moves, results, queen escape:
oracle/hive_oracle.c; tree kernels: oracle/hive_mcts_oracle.c), so that the
GPU orchestrator (hive_neuralnet_amd/orchestrator.py, torch) can be checked
against an independent implementation of the same host logic.

The network is not run here: its outputs for the root and for every
simulation wave, the uniform draws of the Gumbel noise and the Dirichlet
noise are inputs (recorded from the GPU run), in call order.  Top-k ties go
to the lowest slot, as in the GPU counterpart.

Pinning (tests/test_oracle_orchestrator.py): policy_target against the
closed form of its temperature search, _stable_topk's tie order,
immediate_wins against the reference's win detector (golden probe vectors),
_surround against the C oracle's count, `candidate_row` and `qualifying` on
hand-built positions whose qualifying moves and candidate rows were worked
out by hand (tests/orchestrator_cases.py), and `sequential_halving` on
injected candidates, scores and Q whose survivors per round, per-round
simulation counts, wave widths and final choices were worked out in float64
and which each plausible misreading of the rule fails.  The composition in
`run` (root analysis -> candidates -> halving -> policy target) is checked
against the independent torch restatement on recorded GPU plies.
"""
from __future__ import annotations

import math

import numpy as np

from .mcts import MctsOracle

MAX_LEGAL = 256
OFF_TURN, OFF_HEIGHT, OFF_QUEEN = 3412, 2645, 3392
ROUNDS = 4
WAVES = (2, 4, 8, 16)
DIRS = ((1, 0), (1, -1), (0, -1), (-1, 0), (-1, 1), (0, 1))  # (dq, dr) = (col, row) steps


def _neighbours(c):
    row, col = divmod(c, 23)
    out = []
    for dq, dr in DIRS:
        r2, c2 = row + dr, col + dq
        if 0 <= r2 < 23 and 0 <= c2 < 23:
            out.append(r2 * 23 + c2)
    return out


def _turn(s):
    return int(s[OFF_TURN]) | (int(s[OFF_TURN + 1]) << 8)


def _surround(s, colour):
    q = int(s[OFF_QUEEN + 2 * colour]) | (int(s[OFF_QUEEN + 2 * colour + 1]) << 8)
    if q == 0xFFFF:
        return 0
    q = min(max(q, 0), 528)
    return sum(1 for nb in _neighbours(q) if s[OFF_HEIGHT + nb] > 0)


def _stable_topk(x, k):
    order = np.argsort(-x, axis=1, kind="stable")
    return order[:, :k]


def _softmax_rows(x):
    m = x.max(axis=1, keepdims=True)
    e = np.exp((x - m).astype(np.float64))
    return (e / e.sum(axis=1, keepdims=True)).astype(np.float32)


def policy_target(cfg, sampled, valid):
    """_build_policy_target (fnn_mcts_orchestrator.py:144-191)."""
    def soft(temp):
        p = _softmax_rows(sampled / temp)
        p = np.where(valid, p, 0.0).astype(np.float32)
        return (p / np.maximum(p.sum(axis=1, keepdims=True), 1e-12)).astype(np.float32)

    B = sampled.shape[0]
    if not cfg.adaptive_policy_target_temperature:
        t = np.full((B, 1), max(float(cfg.policy_target_temperature), 1e-6), np.float32)
        return soft(t), t[:, 0]
    lo_t = max(float(cfg.policy_target_min_temperature), 1.0)
    hi_t = max(float(cfg.policy_target_max_temperature), lo_t)
    cap = min(max(float(cfg.policy_target_top1_cap), 0.0), 1.0)
    base = np.full((B, 1), lo_t, np.float32)
    probs = soft(base)
    need = probs.max(axis=1, keepdims=True) > cap
    if not need.any() or hi_t <= lo_t:
        return probs, base[:, 0]
    low, high = base.copy(), np.full((B, 1), hi_t, np.float32)
    for _ in range(12):
        mid = ((low + high) * np.float32(0.5)).astype(np.float32)
        sharp = soft(mid).max(axis=1, keepdims=True) > cap
        low = np.where(need & sharp, mid, low)
        high = np.where(need & ~sharp, mid, high)
    final = np.where(need, high, base).astype(np.float32)
    return soft(final), final[:, 0]


def candidate_row(qual, valid, priors, k, reserve):
    """_root_candidate_slots (fnn_mcts_orchestrator.py:411-444) from the
    qualifying mask: `reserve` columns of qualifying slots by prior (-1
    padded), then k columns of the other legal slots by prior, cut to k."""
    B = priors.shape[0]
    rscore = np.where(qual, priors, np.float32(-1e30)).astype(np.float32)
    per_game = np.minimum(qual.sum(axis=1), reserve)
    rorder = _stable_topk(rscore, reserve)
    rvalid = np.arange(reserve)[None, :] < per_game[:, None]
    rcand = np.where(rvalid, rorder, -1).astype(np.int32)
    chosen = np.zeros((B, MAX_LEGAL), bool)
    for g in range(B):
        chosen[g, rorder[g][rvalid[g]]] = True
    fscore = np.where(valid & ~chosen, priors, np.float32(-1e30)).astype(np.float32)
    forder = _stable_topk(fscore, k)
    fkeep = np.maximum(k - per_game, 0)
    fvalid = np.arange(k)[None, :] < fkeep[:, None]
    fcand = np.where(fvalid, forder, -1).astype(np.int32)
    return np.concatenate([rcand, fcand], axis=1)[:, :k]


def sequential_halving(cfg, cand, base, run_round, child_stats):
    """The four halving rounds and the final choice (fnn_mcts_orchestrator.py:650-731).
    cand [B, C] int32 (-1 = none); base [B, 256] float32 Gumbel + legal logits;
    run_round(cand, per_slot, W) runs the simulations of a round; child_stats(cand)
    -> (visits, q) of the candidates' root children.  Returns the chosen slots."""
    B = cand.shape[0]
    rows = np.arange(B)
    per_round = max(1, cfg.num_simulations // ROUNDS)
    for r in range(ROUNDS):
        cvalid = cand >= 0
        C = cand.shape[1]
        W = WAVES[min(r, len(WAVES) - 1)] if cfg.wave_parallel else 1
        run_round(cand, max(1, per_round // C), W)
        if C <= 1:
            continue
        keep_n = np.maximum(cvalid.sum(axis=1) // 2, 1)
        max_keep = C // 2
        visits, q = child_stats(cand)
        sigma = np.float32((cfg.c_visit + visits.max()) * cfg.c_scale)
        b = np.take_along_axis(base, np.maximum(cand, 0).astype(np.int64), axis=1)
        score = np.where(cvalid, (b + sigma * q).astype(np.float32), np.float32(-1e30))
        keep_pos = _stable_topk(score, max_keep)
        ok = np.arange(max_keep)[None, :] < keep_n[:, None]
        cand = np.where(ok, np.take_along_axis(cand, keep_pos, axis=1), -1).astype(np.int32)
    cvalid = cand >= 0
    visits, q = child_stats(cand)
    sigma = np.float32((cfg.c_visit + visits.max()) * cfg.c_scale)
    b = np.take_along_axis(base, np.maximum(cand, 0).astype(np.int64), axis=1)
    final = np.where(cvalid, (b + sigma * q).astype(np.float32), np.float32(-1e30))
    pos = np.argmax(final, axis=1)
    return np.maximum(cand[rows, pos], 0).astype(np.int64)


class SearchPlyOracle:
    def __init__(self, cfg, mcts: MctsOracle | None = None):
        self.cfg = cfg
        self.m = mcts or MctsOracle()
        self.o = self.m.o

    # ---- root analysis -------------------------------------------------
    def immediate_wins(self, states, legal, n):  # :446-493
        wins = np.full(states.shape[0], -1, np.int64)
        for g in range(states.shape[0]):
            white = _turn(states[g]) % 2 == 0
            for i in range(int(n[g])):
                r = int(self.o.apply_move(states[g], legal[g, i])[3415])
                if (r == 1 and white) or (r == 2 and not white):
                    wins[g] = i
                    break
        return wins

    def qualifying(self, states, legal, n):  # :339-382
        qual = np.zeros((states.shape[0], MAX_LEGAL), bool)
        for g in range(states.shape[0]):
            before = _surround(states[g], (_turn(states[g]) + 1) & 1)
            for i in range(int(n[g])):
                child = self.o.apply_move(states[g], legal[g, i])
                after = _surround(child, _turn(child) & 1)
                ok = after > before
                if ok and self.cfg.queen_surround_reserve_immobile_only:
                    ok = not self.o.queen_escape(child)
                qual[g, i] = ok
        return qual

    def candidates(self, states, legal, n, priors, legal_logits, allowed):  # :384-444
        cfg = self.cfg
        B = states.shape[0]
        k = min(int(cfg.max_num_considered_actions), MAX_LEGAL)
        valid = (np.arange(MAX_LEGAL)[None, :] < n[:, None]) & allowed
        reserve = min(int(cfg.queen_surround_reserve_slots), k)
        if reserve <= 0:
            raise NotImplementedError("reserve_slots <= 0 draws a second Gumbel sample")
        qual = self.qualifying(states, legal, n)
        return candidate_row(qual, valid, priors, k, reserve)

    # ---- search --------------------------------------------------------
    def root_stats(self, t, slots):  # _gather_root_candidate_stats :1072-1096
        B = slots.shape[0]
        rows = np.arange(B)
        root = t["root_node"]
        fc = t["first_child"][rows, root].astype(np.int64)
        nc = t["num_children"][rows, root].astype(np.int64)
        s = slots.astype(np.int64)
        valid = (s >= 0) & (fc[:, None] >= 0) & (s < nc[:, None])
        idx = np.clip(fc[:, None] + np.maximum(s, 0), 0, t["visit_count"].shape[1] - 1)
        vr = t["visit_count"][rows[:, None], idx]
        tr = t["total_value"][rows[:, None], idx]
        visits = np.where(valid, vr, 0)
        q = np.where(valid & (vr > int(self.cfg.root_q_min_visits)),
                     (-tr / np.maximum(vr, 1).astype(np.float32)).astype(np.float32), np.float32(0))
        return visits, q.astype(np.float32)

    def run(self, t, states, active, legal, n, root_eval, uniforms, noise, wave_evals, forced_uniforms=None):
        """One ply.  root_eval = (priors, root values, child_q); uniforms = the
        [B, 256] Gumbel draws; noise = the [B, max_children] Dirichlet rows;
        wave_evals = per simulation wave (priors, values, child_q);
        forced_uniforms = the [B] draws of the random move of games the root
        probe leaves without a safe move (short_forced_win_probe only).
        Returns (chosen slot, policy, slot visits); t is updated in place."""
        cfg = self.cfg
        B = states.shape[0]
        slot = np.arange(MAX_LEGAL)[None, :]
        valid = slot < n[:, None]
        has_actions = active & (n > 0)
        priors, _, child_q = (np.array(a, np.float32, copy=True) for a in root_eval)
        allowed = valid
        forced = np.zeros(B, bool)
        if cfg.short_forced_win_probe:  # _analyze_short_tactics :527-545, used at :611-617
            wins, allowed_u8, forced_u8 = self.o.batch_root_tactical_probe(
                states, legal, n, priors, cfg.probe_win_in_one, cfg.probe_check_opponent_wins, cfg.probe_win_in_two)
            allowed = (allowed_u8 != 0) & valid
            forced = (forced_u8 != 0) & has_actions
        else:
            wins = self.immediate_wins(states, legal, n)
        has_win = wins >= 0
        if has_win.any():
            priors[:] = 0.0
            priors[has_win, wins[has_win]] = 1.0
            child_q[:] = 0.0
        search = has_actions & ~has_win & ~forced
        legal_logits = np.where(allowed, np.log(np.maximum(priors, np.float32(1e-20))), np.float32(-1e30))
        legal_logits = legal_logits.astype(np.float32)
        u = np.clip(uniforms.astype(np.float32), np.float32(1e-4), np.float32(1 - 1e-4))
        gumbel = np.where(allowed, -np.log(-np.log(u)), np.float32(-1e30)).astype(np.float32)
        cand_all = self.candidates(states, legal, n, priors, legal_logits, allowed)
        # root expansion (:879-902) and noise (:904-925)
        rows = np.arange(B)
        fc = t["first_child"][rows, t["root_node"]]
        needs = (fc < 0) & search
        if needs.any():
            leaf = np.where(needs, t["root_node"], -1).astype(np.int32)
            res = states[:, 3415].astype(np.int32)
            self.m.expand_dense(t, np.ascontiguousarray(child_q), leaf, states, legal, n.astype(np.int32),
                                np.ascontiguousarray(priors), res)
        self.m.root_noise(t, noise, t["root_node"], cfg.dirichlet_epsilon, 1.0)
        slot_visits = np.zeros((B, MAX_LEGAL), np.int32)
        probs = np.zeros((B, MAX_LEGAL), np.float32)
        chosen = np.zeros(B, np.int64)
        waves = iter(wave_evals)
        if search.any():
            cand = cand_all.astype(np.int32)
            cvalid = np.take_along_axis(valid, np.maximum(cand, 0), axis=1) & (cand >= 0)
            cand = np.where(cvalid, cand, -1).astype(np.int32)
            active8 = search.astype(np.int8)

            def run_round(cand, per_slot, W):
                for w in range(math.ceil(per_slot / W)):
                    ww = min(W, per_slot - w * W)
                    leaf, paths, plen, vl, vlen = self.m.select_slots(
                        t, active8, t["root_node"], cand, MAX_LEGAL, cfg.c_puct, ww)
                    leaves = np.zeros((leaf.shape[0], 3424), np.uint8)
                    self.m.replay(states, leaves, paths, plen, leaf)
                    res = leaves[:, 3415].astype(np.int32)
                    lm, ln, _, _ = self.o.batch_legal_features_actions(leaves, want_features=False,
                                                                       want_actions=False)
                    p2, v2, q2 = next(waves)
                    self.m.expand_backprop_dense(t, np.ascontiguousarray(q2, np.float32), leaf, leaves, lm, ln,
                                                 np.ascontiguousarray(p2, np.float32), res,
                                                 np.ascontiguousarray(v2, np.float32), vl, vlen)
                return per_slot * cand.shape[1] * B

            chosen = sequential_halving(cfg, cand, (gumbel + legal_logits).astype(np.float32), run_round,
                                        lambda c: self.root_stats(t, c))
            slot_visits, slot_q = self.root_stats(t, np.broadcast_to(slot, (B, MAX_LEGAL)))
            visited = (slot_visits > 0) & valid
            max_n = slot_visits.astype(np.float32).max(axis=1, keepdims=True)
            sampled = np.where(visited, (legal_logits + (cfg.c_visit + max_n) * cfg.c_scale * slot_q),
                               np.float32(-1e30)).astype(np.float32)
            probs, _ = policy_target(cfg, sampled, valid)
        if has_win.any():
            slot_visits[has_win] = 0
            slot_visits[has_win, wins[has_win]] = cfg.num_simulations
            probs[has_win] = 0.0
            probs[has_win, wins[has_win]] = 1.0
            chosen = np.where(has_win, wins, chosen)
        if forced.any():  # :768-776
            rnd = (np.asarray(forced_uniforms, np.float32) * np.maximum(n, 1).astype(np.float32)).astype(np.int64)
            chosen = np.where(forced, rnd, chosen)
            probs[forced] = 0.0
        return chosen, probs, slot_visits
