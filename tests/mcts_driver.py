"""A small Gumbel-style search driver over the MCTS tree entry points.

Test helper.  It runs the reference orchestrator's call sequence
(hive_fnn/fnn_mcts_orchestrator.py:645-711,896-925,982-1055): root expansion
with dense priors, root noise, then waves of root-slot selection, replay,
results, legal lists, expansion + backup -- with the network replaced by
seeded synthetic outputs computed on the host (record-and-replay), so the
CPU oracle and the GPU engine receive identical inputs and their trees can
be compared array by array.
"""
from __future__ import annotations

import numpy as np

from oracle.mcts import TREE_KEYS, MctsOracle, new_tree

MAX_LEGAL = 256


def synthetic_eval(rng, n, total):
    """Softmax priors over legal slots, values and child Q in [-1, 1]."""
    valid = np.arange(MAX_LEGAL)[None, :] < n[:total, None]
    logits = rng.standard_normal((total, MAX_LEGAL))
    logits = np.where(valid, logits, -np.inf)
    mx = np.max(np.where(valid, logits, -1e300), axis=1, keepdims=True)
    e = np.where(valid, np.exp(logits - mx), 0.0)
    s = e.sum(axis=1, keepdims=True)
    pri = np.where(s > 0, e / np.where(s > 0, s, 1), 0.0).astype(np.float32)
    vals = rng.uniform(-1, 1, total).astype(np.float32)
    cq = np.where(valid, rng.uniform(-1, 1, (total, MAX_LEGAL)), 0.0).astype(np.float32)
    return np.ascontiguousarray(pri), vals, np.ascontiguousarray(cq)


class OracleEngine:
    def __init__(self):
        self.m = MctsOracle()
        self.o = self.m.o

    def tree(self, B, M):
        return new_tree(B, M)

    def to_np(self, t):
        return t

    def legal(self, states):
        m, n, _, _ = self.o.batch_legal_features_actions(states, want_features=False, want_actions=False)
        return m, n

    def expand_dense(self, t, cq, leaf, states, legal, n, pri, results):
        return self.m.expand_dense(t, cq, leaf, states, legal, n, pri, results)

    def root_noise(self, t, noise, eps):
        self.m.root_noise(t, noise, t["root_node"], eps)

    def select_slots(self, t, active, slots, max_root, c_puct, W, det=False, sigma=4.0, qp=0.0):
        return self.m.select_slots(t, active, t["root_node"], slots, max_root, c_puct, W, det, sigma, qp)

    def select_mask(self, t, active, alive, c_puct, W, det=False, sigma=4.0, qp=0.0):
        return self.m.select_mask(t, active, t["root_node"], alive, c_puct, W, det, sigma, qp)

    def replay(self, roots, paths, plen, leaf):
        leaves = np.zeros((leaf.shape[0], 3424), np.uint8)
        self.m.replay(roots, leaves, paths, plen, leaf)
        return leaves

    def expand_backprop(self, t, cq, leaf, states, legal, n, pri, results, vals, vl, vlen, qp=0.0):
        self.m.expand_backprop_dense(t, cq, leaf, states, legal, n, pri, results, vals, vl, vlen, qp)


def _oracle_legacy(cls):
    def select_legacy(self, t, active, c_puct, W):
        return self.m.select_legacy(t, active, t["root_node"], c_puct, W)

    def expand_legacy(self, t, leaf, states, legal, n, probs, results):
        return self.m.expand_legacy(t, leaf, states, legal, n, probs, results)

    def backprop_legacy(self, t, leaf, vals, vl, vlen, was):
        self.m.backprop_legacy(t, leaf, vals, vl, vlen, was)

    def expand_backprop_legacy(self, t, leaf, states, legal, n, probs, results, vals, vl, vlen):
        self.m.expand_backprop_legacy(t, leaf, states, legal, n, probs, results, vals, vl, vlen)

    def extract_policy(self, t, move_numbers, temperature, temp_drop, pruning):
        return self.m.extract_policy(t, move_numbers, t["root_node"], temperature, temp_drop, pruning)

    def legal_mask(self, states):
        legal, n = self.legal(states)
        return self.m.legal_mask(states, legal, n), n

    for f in (select_legacy, expand_legacy, backprop_legacy, expand_backprop_legacy, extract_policy, legal_mask):
        setattr(cls, f.__name__, f)
    return cls


_oracle_legacy(OracleEngine)


class GpuEngine:
    """Same interface over hive_neuralnet_amd.hive_gpu (all device work through the C-ABI)."""

    def __init__(self):
        import torch
        from hive_neuralnet_amd import hive_gpu
        self.torch = torch
        self.ext = hive_gpu.load_extension()

    def c(self, a):
        return self.torch.from_numpy(np.ascontiguousarray(a)).cuda()

    def tree(self, B, M):
        return {k: self.c(v) for k, v in new_tree(B, M).items()}

    def to_np(self, t):
        return {k: v.cpu().numpy() for k, v in t.items()}

    def args(self, t):
        return [t["visit_count"], t["total_value"], t["prior"], t["parent_idx"], t["virtual_q_penalty"],
                t["move_bytes"], t["action_idx"], t["first_child"], t["num_children"], t["is_terminal"],
                t["terminal_value"], t["node_count"]]

    def M(self, t):
        return t["visit_count"].shape[1]

    def legal(self, states):
        m, n = self.ext.generate_legal_moves_batch(self.c(states), states.shape[0])
        return m.cpu().numpy(), n.cpu().numpy()

    def expand_dense(self, t, cq, leaf, states, legal, n, pri, results):
        B = t["node_count"].shape[0]
        was = self.ext.mcts_expand_dense_priors_batch(
            *self.args(t), t["child_init_q"], self.c(cq), self.c(leaf), self.c(states), self.c(legal), self.c(n),
            self.c(pri), self.c(results), B, leaf.shape[0], self.M(t))
        return was.cpu().numpy()

    def root_noise(self, t, noise, eps):
        B = t["node_count"].shape[0]
        self.ext.mcts_apply_root_noise(*self.args(t), self.c(noise.astype(np.float32)), t["root_node"],
                                       noise.shape[1], eps, 1.0, B, self.M(t))

    def select_slots(self, t, active, slots, max_root, c_puct, W, det=False, sigma=4.0, qp=0.0):
        B, C = slots.shape
        out = self.ext.mcts_select_with_root_slots_batch(
            *self.args(t), t["child_init_q"], self.c(active.astype(np.int8)), t["root_node"],
            self.c(slots.astype(np.int32)), C, max_root, c_puct, B, W, self.M(t), det, sigma, qp)
        return tuple(o.cpu().numpy() for o in out)

    def select_mask(self, t, active, alive, c_puct, W, det=False, sigma=4.0, qp=0.0):
        B, max_root = alive.shape
        out = self.ext.mcts_select_with_root_mask_batch(
            *self.args(t), t["child_init_q"], self.c(active.astype(np.int8)), t["root_node"],
            self.c(alive.astype(np.int8)), max_root, c_puct, B, W, self.M(t), det, sigma, qp)
        return tuple(o.cpu().numpy() for o in out)

    def replay(self, roots, paths, plen, leaf):
        total = leaf.shape[0]
        leaves = self.torch.zeros((total, 3424), dtype=self.torch.uint8, device="cuda")
        self.ext.mcts_replay_batch(self.c(roots), leaves, self.c(paths), self.c(plen), self.c(leaf),
                                   roots.shape[0], total)
        return leaves.cpu().numpy()

    def expand_backprop(self, t, cq, leaf, states, legal, n, pri, results, vals, vl, vlen, qp=0.0):
        B = t["node_count"].shape[0]
        self.ext.mcts_expand_and_backprop_dense_priors_batch(
            *self.args(t), t["child_init_q"], self.c(cq), self.c(leaf), self.c(states), self.c(legal), self.c(n),
            self.c(pri), self.c(results), self.c(vals), self.c(vl), self.c(vlen), B, leaf.shape[0], self.M(t), qp)


def _gpu_legacy(cls):
    def select_legacy(self, t, active, c_puct, W):
        B = t["node_count"].shape[0]
        out = self.ext.mcts_select_batch(*self.args(t), self.c(active.astype(np.int8)), t["root_node"], c_puct, B, W,
                                         self.M(t))
        return tuple(o.cpu().numpy() for o in out)

    def expand_legacy(self, t, leaf, states, legal, n, probs, results):
        B = t["node_count"].shape[0]
        was = self.ext.mcts_expand_batch(*self.args(t), self.c(leaf), self.c(states), self.c(legal), self.c(n),
                                         self.c(probs), self.c(results), B, leaf.shape[0], self.M(t))
        return was.cpu().numpy()

    def backprop_legacy(self, t, leaf, vals, vl, vlen, was):
        B = t["node_count"].shape[0]
        self.ext.mcts_backprop_batch(*self.args(t), self.c(leaf), self.c(vals), self.c(vl), self.c(vlen), self.c(was),
                                     B, leaf.shape[0], self.M(t))

    def expand_backprop_legacy(self, t, leaf, states, legal, n, probs, results, vals, vl, vlen):
        B = t["node_count"].shape[0]
        self.ext.mcts_expand_and_backprop_batch(*self.args(t), self.c(leaf), self.c(states), self.c(legal),
                                                self.c(n), self.c(probs), self.c(results), self.c(vals), self.c(vl),
                                                self.c(vlen), B, leaf.shape[0], self.M(t))

    def extract_policy(self, t, move_numbers, temperature, temp_drop, pruning):
        B = t["node_count"].shape[0]
        return self.ext.mcts_extract_policy_batch(*self.args(t), self.c(move_numbers.astype(np.int32)),
                                                  t["root_node"], temperature, temp_drop, pruning, B,
                                                  self.M(t)).cpu().numpy()

    def legal_mask(self, states):
        m, n = self.ext.generate_legal_mask_batch(self.c(states), states.shape[0])
        return m.cpu().numpy(), n.cpu().numpy()

    for f in (select_legacy, expand_legacy, backprop_legacy, expand_backprop_legacy, extract_policy, legal_mask):
        setattr(cls, f.__name__, f)
    return cls


_gpu_legacy(GpuEngine)


def action_probs(rng, total):
    """Synthetic [total, 85834] action-space priors (every entry positive)."""
    return np.ascontiguousarray(rng.uniform(0.01, 1.0, (total, 85834)).astype(np.float32))


def run_search_legacy(engine, roots, *, seed=3, M=4096, W=2, waves=5, c_puct=1.25, split=False):
    """The legacy engine's loop (hive_gpu/gpu_native_mcts.py:300-365): root
    expansion from action-space priors, then waves of PUCT select / replay /
    legal / expand + backup (separate expand and backup kernels when split),
    then the policies for three temperatures.  Returns (tree, records, policies)."""
    rng = np.random.default_rng(seed)
    B = roots.shape[0]
    t = engine.tree(B, M)
    legal, n = engine.legal(roots)
    results = roots[:, 3415].astype(np.int32)
    active = (results == 0) & (n > 0)
    leaf0 = np.where(active, 0, -1).astype(np.int32)
    was = engine.expand_legacy(t, leaf0, roots, legal, n, action_probs(rng, B), results)
    records = [{"was_root": was}]
    for _ in range(waves):
        leaf, paths, plen, vl, vlen = engine.select_legacy(t, active, c_puct, W)
        leaves = engine.replay(roots, paths, plen, leaf)
        res = leaves[:, 3415].astype(np.int32)
        lm, ln = engine.legal(leaves)
        probs = action_probs(rng, leaf.shape[0])
        vals = rng.uniform(-1, 1, leaf.shape[0]).astype(np.float32)
        rec = {"leaf": leaf, "paths": paths, "plen": plen, "vl": vl, "vlen": vlen, "leaves": leaves}
        if split:
            rec["was"] = engine.expand_legacy(t, leaf, leaves, lm, ln, probs, res)
            engine.backprop_legacy(t, leaf, vals, vl, vlen, rec["was"])
        else:
            engine.expand_backprop_legacy(t, leaf, leaves, lm, ln, probs, res, vals, vl, vlen)
        records.append(rec)
    mn = np.arange(B, dtype=np.int32) % 3 * 10  # 0, 10, 20: the last group past temp_drop 15
    policies = [engine.extract_policy(t, mn, temp, 15, prune) for temp, prune in ((1.0, 0.0), (1.0, 0.2),
                                                                                  (0.5, 0.0))]
    return engine.to_np(t), records, policies


def run_search(engine, roots, *, seed=1, M=4096, C=4, W=2, waves=6, c_puct=1.25, eps=0.25, mode="slots", dup=False,
               det=False, sigma=4.0, qp=0.0):
    """Root expand + noise + `waves` select/replay/legal/expand-backup rounds
    (det: completed-Q descent below the root with q penalty qp, as the
    orchestrator's deterministic_non_root mode).

    Returns (final tree as numpy, list of per-wave records)."""
    rng = np.random.default_rng(seed)
    B = roots.shape[0]
    t = engine.tree(B, M)
    start_visits = engine.to_np(t)["visit_count"].copy()
    legal, n = engine.legal(roots)
    pri, _, cq = synthetic_eval(rng, n, B)
    results = roots[:, 3415].astype(np.int32)
    active = (results == 0) & (n > 0)
    leaf0 = np.where(active, 0, -1).astype(np.int32)
    was = engine.expand_dense(t, cq, leaf0, roots, legal, n, pri, results)
    nc = np.maximum(n, 1)
    noise = np.zeros((B, int(nc.max())), np.float32)
    for i in range(B):
        noise[i, : n[i]] = rng.dirichlet([0.3] * max(1, n[i]))[: n[i]]
    engine.root_noise(t, noise, eps)
    order = np.argsort(-pri, axis=1, kind="stable")[:, :C]
    slots = np.where(np.arange(C)[None, :] < n[:, None], order, -1).astype(np.int32)
    if dup:  # every third game forces two candidates into the same root child
        slots[::3, C - 1] = slots[::3, 0]
    alive = np.zeros((B, MAX_LEGAL), np.int8)
    for i in range(B):
        alive[i, slots[i][slots[i] >= 0]] = 1
    records = [{"was_root": was, "post_visits": engine.to_np(t)["visit_count"].copy(), "start": start_visits}]
    for _ in range(waves):
        if mode == "slots":
            leaf, paths, plen, vl, vlen = engine.select_slots(t, active, slots, MAX_LEGAL, c_puct, W, det, sigma, qp)
        else:
            leaf, paths, plen, vl, vlen = engine.select_mask(t, active, alive, c_puct, W, det, sigma, qp)
        leaves = engine.replay(roots, paths, plen, leaf)
        res = leaves[:, 3415].astype(np.int32)
        lm, ln = engine.legal(leaves)
        p2, v2, q2 = synthetic_eval(rng, ln, leaf.shape[0])
        mid = engine.to_np(t)
        mid_visits, mid_total = mid["visit_count"].copy(), mid["total_value"].copy()
        engine.expand_backprop(t, q2, leaf, leaves, lm, ln, p2, res, v2, vl, vlen, qp)
        post_visits = engine.to_np(t)["visit_count"].copy()
        records.append({"leaf": leaf, "paths": paths, "plen": plen, "vl": vl, "vlen": vlen, "leaves": leaves,
                        "mid_visits": mid_visits, "mid_total": mid_total, "post_visits": post_visits})
    return engine.to_np(t), records


def tree_equal(a, b):
    bad = []
    for k in TREE_KEYS + ["root_node"]:
        x, y = a[k], b[k]
        if x.dtype == np.float32:
            x, y = x.view(np.uint32), y.view(np.uint32)
        if not np.array_equal(x, y):
            bad.append(k)
    return bad


# Completed-Q descent known answers (deterministic_completed_q_child,
# mcts_tree.cuh:77-143).  Each case: the children of the forced root child
# as (N, W, prior, child_init_q, virtual_q_penalty), the forced child's own
# N, and the child the rule picks.  The choice was computed by hand in float64
# (pi0 = softmax_c(log max(prior, 1e-20) + 4 q_c), q = -W/N, or child_init_q
# when N = 0, minus the virtual-Q penalty; score = pi0 - N / (1 + sum N)):
#   case 0 scores  0.049245  0.019896  0.082595  0.014931 -> child 2 (margin 0.033)
#   case 1 scores  0.389749 -0.429166  0.150528           -> child 0
#   case 2 scores -0.108718  0.348829 -0.115111           -> child 1
# Each plausible misreading picks another child: +W/N (case 0 -> 0, case 1 -> 1,
# case 2 -> 2); 0 or -child_init_q for unvisited children (case 0 -> 0);
# no penalty or +penalty (case 0 -> 3, case 2 -> 0); no log prior (case 0 -> 3);
# the parent's N in the denominator (case 0 -> 3); N / sum N (case 0 -> 0);
# pi0 + N/(1 + sum N) (case 0 -> 3); sigma 1 instead of 4 (case 0 -> 0, case 1 -> 2).
COMPLETED_Q_CASES = [
    ([(0, 0.0, 0.4, -0.82, 0.0), (0, 0.0, 0.1, -0.7, 0.0), (2, -0.62, 0.1, 0.0, 0.25), (3, -2.36, 0.05, 0.0, 0.5)],
     65, 2),
    ([(4, -2.0, 0.3, 0.0, 0.0), (4, 2.0, 0.3, 0.0, 0.0), (0, 0.0, 0.4, 0.0, 0.0)], 8, 0),
    ([(3, -1.5, 0.4, 0.0, 0.35), (3, -1.2, 0.4, 0.0, 0.0), (1, 0.5, 0.2, 0.0, 0.0)], 7, 1),
]


def completed_q_trees(M=16):
    """One game per case: root 0 -> forced child 1 -> children 2.. (unexpanded).
    Returns (tree, expected leaf node per game)."""
    B = len(COMPLETED_Q_CASES)
    t = new_tree(B, M)
    want = []
    for g, (kids, parent_n, pick) in enumerate(COMPLETED_Q_CASES):
        t["first_child"][g, 0], t["num_children"][g, 0] = 1, 1
        t["parent_idx"][g, 1] = 0
        t["prior"][g, 1] = 1.0
        t["visit_count"][g, 0] = t["visit_count"][g, 1] = parent_n
        t["first_child"][g, 1], t["num_children"][g, 1] = 2, len(kids)
        for i, (n, w, p, ciq, vq) in enumerate(kids):
            u = 2 + i
            t["visit_count"][g, u], t["total_value"][g, u], t["prior"][g, u] = n, w, p
            t["child_init_q"][g, u], t["virtual_q_penalty"][g, u] = ciq, vq
            t["parent_idx"][g, u] = 1
            t["move_bytes"][g, u] = [2, 0, 0, 0, 0, 0]
        t["move_bytes"][g, 1] = [2, 0, 0, 0, 0, 0]
        t["node_count"][g] = 2 + len(kids)
        want.append(2 + pick)
    return t, np.array(want, np.int32)


def record_wave_evaluations(monkeypatch, evals):
    """Append each native simulation wave's (priors, values, child Q) to
    `evals` (numpy copies), as a recorded _eval_states call would: the
    orchestrator's waves run as one library call (WavePlan.run) whose
    evaluation outputs stay in the plan's buffers."""
    from hive_neuralnet_amd import hive_gpu
    real_run = hive_gpu.WavePlan.run

    def run(plan, *a, **k):
        out = real_run(plan, *a, **k)
        T = int(a[7]) * int(a[4]) * plan.B
        evals.append(tuple(x[:T].detach().cpu().numpy().copy() for x in (plan.priors, plan.values, plan.child_q)))
        return out
    monkeypatch.setattr(hive_gpu.WavePlan, "run", run)

