"""ctypes wrapper of the MCTS tree oracle (oracle/hive_mcts_oracle.c).

TEST INFRASTRUCTURE ONLY.  Trees are dicts of numpy arrays with the
reference's names (hive_fnn/fnn_mcts_orchestrator.py:195-214 layout).
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import FEAT_DIM, MAX_LEGAL, STATE_BYTES, Oracle  # noqa: F401

DEPTH = 128


class _OrTree(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("vc", "tv", "pr", "pa", "vq", "mb", "ai", "fc", "nc", "it", "tval",
                                               "cnt", "ciq")] + [("M", ctypes.c_int64)]


TREE_KEYS = ["visit_count", "total_value", "prior", "parent_idx", "virtual_q_penalty", "move_bytes", "action_idx",
             "first_child", "num_children", "is_terminal", "terminal_value", "node_count", "child_init_q"]


def new_tree(B: int, M: int) -> dict:
    """Fresh trees as the reference's _alloc_tree + _reset_tree leave them."""
    return {
        "visit_count": np.zeros((B, M), np.int32),
        "total_value": np.zeros((B, M), np.float32),
        "prior": np.zeros((B, M), np.float32),
        "virtual_q_penalty": np.zeros((B, M), np.float32),
        "parent_idx": np.full((B, M), -1, np.int32),
        "move_bytes": np.zeros((B, M, 6), np.uint8),
        "action_idx": np.full((B, M), -1, np.int32),
        "first_child": np.full((B, M), -1, np.int32),
        "num_children": np.zeros((B, M), np.int32),
        "is_terminal": np.zeros((B, M), np.int8),
        "terminal_value": np.zeros((B, M), np.float32),
        "node_count": np.ones((B,), np.int32),
        "root_node": np.zeros((B,), np.int32),
        "child_init_q": np.zeros((B, M), np.float32),
    }


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


class MctsOracle:
    def __init__(self, oracle: Oracle | None = None):
        self.o = oracle or Oracle()
        self.lib = self.o.lib

    def _tree(self, t: dict) -> _OrTree:
        for k in TREE_KEYS:
            assert t[k].flags.c_contiguous, k
        M = t["visit_count"].shape[1]
        return _OrTree(_p(t["visit_count"]), _p(t["total_value"]), _p(t["prior"]), _p(t["parent_idx"]),
                       _p(t["virtual_q_penalty"]), _p(t["move_bytes"]), _p(t["action_idx"]), _p(t["first_child"]),
                       _p(t["num_children"]), _p(t["is_terminal"]), _p(t["terminal_value"]), _p(t["node_count"]),
                       _p(t["child_init_q"]), M)

    @staticmethod
    def _outs(T):
        return (np.zeros(T, np.int32), np.zeros((T, DEPTH, 6), np.uint8), np.zeros(T, np.int32),
                np.zeros((T, DEPTH), np.int32), np.zeros(T, np.int32))

    def select_slots(self, t, game_active, root_nodes, root_slots, max_root, c_puct, W, det=False, sigma=4.0,
                     q_penalty=0.0):
        B, C = root_slots.shape
        out = self._outs(W * C * B)
        tr = self._tree(t)
        self.lib.or_mcts_select_slots(
            ctypes.byref(tr), _p(np.ascontiguousarray(game_active, np.int8)),
            _p(np.ascontiguousarray(root_nodes, np.int32)), _p(np.ascontiguousarray(root_slots, np.int32)),
            ctypes.c_int(C), ctypes.c_int(max_root), ctypes.c_float(c_puct), ctypes.c_int64(B), ctypes.c_int(W),
            ctypes.c_int(1 if det else 0), ctypes.c_float(sigma), ctypes.c_float(q_penalty), *[_p(o) for o in out])
        return out

    def select_mask(self, t, game_active, root_nodes, alive, c_puct, W, det=False, sigma=4.0, q_penalty=0.0):
        B, max_root = alive.shape
        out = self._outs(W * B)
        tr = self._tree(t)
        self.lib.or_mcts_select_mask(
            ctypes.byref(tr), _p(np.ascontiguousarray(game_active, np.int8)),
            _p(np.ascontiguousarray(root_nodes, np.int32)), _p(np.ascontiguousarray(alive, np.int8)),
            ctypes.c_int(max_root), ctypes.c_float(c_puct), ctypes.c_int64(B), ctypes.c_int(W),
            ctypes.c_int(1 if det else 0), ctypes.c_float(sigma), ctypes.c_float(q_penalty), *[_p(o) for o in out])
        return out

    def replay(self, roots, leaves, paths, plen, leaf):
        B = roots.shape[0]
        self.lib.or_mcts_replay(_p(roots), ctypes.c_int64(B), _p(leaves), _p(paths), _p(plen), _p(leaf),
                                ctypes.c_int64(leaves.shape[0]))

    def expand_dense(self, t, child_q, leaf, states, legal, nlegal, priors, results):
        B = t["node_count"].shape[0]
        total = leaf.shape[0]
        was = np.zeros(total, np.int8)
        tr = self._tree(t)
        self.lib.or_mcts_expand_dense(ctypes.byref(tr), _p(child_q), _p(leaf), _p(states), _p(legal), _p(nlegal),
                                      _p(priors), _p(results), ctypes.c_int64(B), ctypes.c_int64(total), _p(was))
        return was

    def expand_backprop_dense(self, t, child_q, leaf, states, legal, nlegal, priors, results, values, vl, vlen,
                              q_penalty=0.0):
        B = t["node_count"].shape[0]
        total = leaf.shape[0]
        tr = self._tree(t)
        self.lib.or_mcts_expand_backprop_dense(
            ctypes.byref(tr), _p(child_q), _p(leaf), _p(states), _p(legal), _p(nlegal), _p(priors), _p(results),
            _p(values), _p(vl), _p(vlen), ctypes.c_float(q_penalty), ctypes.c_int64(B), ctypes.c_int64(total))

    def root_noise(self, t, noise, root_nodes, eps, temp=1.0):
        B, pad = noise.shape
        tr = self._tree(t)
        self.lib.or_mcts_root_noise(ctypes.byref(tr), _p(np.ascontiguousarray(noise, np.float32)),
                                    _p(np.ascontiguousarray(root_nodes, np.int32)), ctypes.c_int(pad),
                                    ctypes.c_float(eps), ctypes.c_float(temp), ctypes.c_int64(B))

    # ---- legacy action-space engine (mcts_tree.cuh:205-687) ----------------
    def select_legacy(self, t, game_active, root_nodes, c_puct, W):
        B = t["node_count"].shape[0]
        out = self._outs(W * B)
        tr = self._tree(t)
        self.lib.or_mcts_select_legacy(
            ctypes.byref(tr), _p(np.ascontiguousarray(game_active, np.int8)),
            _p(np.ascontiguousarray(root_nodes, np.int32)), ctypes.c_float(c_puct), ctypes.c_int64(B), ctypes.c_int(W),
            *[_p(o) for o in out])
        return out

    def expand_legacy(self, t, leaf, states, legal, nlegal, probs, results):
        B = t["node_count"].shape[0]
        total = leaf.shape[0]
        was = np.zeros(total, np.int8)
        tr = self._tree(t)
        self.lib.or_mcts_expand_legacy(ctypes.byref(tr), _p(leaf), _p(states), _p(legal), _p(nlegal), _p(probs),
                                       _p(results), ctypes.c_int64(B), ctypes.c_int64(total), _p(was))
        return was

    def backprop_legacy(self, t, leaf, values, vl, vlen, was):
        B = t["node_count"].shape[0]
        tr = self._tree(t)
        self.lib.or_mcts_backprop_legacy(ctypes.byref(tr), _p(leaf), _p(values), _p(vl), _p(vlen), _p(was),
                                         ctypes.c_int64(B), ctypes.c_int64(leaf.shape[0]))

    def expand_backprop_legacy(self, t, leaf, states, legal, nlegal, probs, results, values, vl, vlen):
        B = t["node_count"].shape[0]
        tr = self._tree(t)
        self.lib.or_mcts_expand_backprop_legacy(ctypes.byref(tr), _p(leaf), _p(states), _p(legal), _p(nlegal),
                                                _p(probs), _p(results), _p(values), _p(vl), _p(vlen),
                                                ctypes.c_int64(B), ctypes.c_int64(leaf.shape[0]))

    def extract_policy(self, t, move_numbers, root_nodes, temperature, temp_drop, pruning):
        B = t["node_count"].shape[0]
        out = np.zeros((B, 85834), np.float32)
        tr = self._tree(t)
        self.lib.or_mcts_extract_policy(ctypes.byref(tr), _p(np.ascontiguousarray(move_numbers, np.int32)),
                                        _p(np.ascontiguousarray(root_nodes, np.int32)), ctypes.c_float(temperature),
                                        ctypes.c_int(temp_drop), ctypes.c_float(pruning), ctypes.c_int64(B), _p(out))
        return out

    def legal_mask(self, states, legal, nlegal):
        B = states.shape[0]
        out = np.zeros((B, 85834), np.float32)
        self.lib.or_legal_mask(_p(np.ascontiguousarray(states)), _p(np.ascontiguousarray(legal)),
                               _p(np.ascontiguousarray(nlegal, np.int32)), ctypes.c_int64(B), _p(out))
        return out
