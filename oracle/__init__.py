"""CPU oracle for the batched Hive engine (TEST INFRASTRUCTURE ONLY).

This package is the parity checker.  Only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg import it.  The product
(``hive_neuralnet_amd``) never does: its HIP path must stand on its own and
fail loudly when its library is missing.

Two CPU engines live here:

* ``Oracle`` -- this repository's own C restatement (``oracle/hive_oracle.c``)
  of the reference semantics, built by ``make -C oracle``.
* ``Reference`` -- the reference's own ``hive_gpu/csrc/cpu_native.cpp``
  compiled where it lies (``oracle/ref_capi.cpp``, ``make -C oracle ref``),
  available only where ``oracle/_ref/libhive_ref.so`` was built.  It writes
  the golden vectors and pins the restatement.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
STATE_BYTES = 3424
MOVE_BYTES = 6
MAX_LEGAL = 256
FEAT_DIM = 122

_u8p = ctypes.POINTER(ctypes.c_uint8)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_f32p = ctypes.POINTER(ctypes.c_float)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_i16p = ctypes.POINTER(ctypes.c_int16)


def _ptr(a, t):
    return a.ctypes.data_as(t) if a is not None else ctypes.cast(None, t)


def build(ref: bool = False) -> None:
    """Compile the oracle (and the reference shim when asked) in place."""
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)
    if ref:
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


def default_threads() -> int:
    n = os.cpu_count() or 1
    return max(1, min(n, 16))


class _Engine:
    prefix = ""

    def __init__(self, lib):
        self.lib = lib

    def _f(self, name):
        return getattr(self.lib, self.prefix + name)

    # single-state API -------------------------------------------------
    def init_state(self, mask: int = 0) -> np.ndarray:
        s = np.zeros(STATE_BYTES, np.uint8)
        self._f("init_state")(_ptr(s, _u8p), int(mask))
        return s

    def apply_move(self, state: np.ndarray, move6) -> np.ndarray:
        s = np.array(state, dtype=np.uint8, copy=True)
        m = np.ascontiguousarray(np.asarray(move6, dtype=np.uint8).reshape(6))
        self._f("apply_move")(_ptr(s, _u8p), _ptr(m, _u8p))
        return s

    def legal_moves(self, state: np.ndarray):
        s = np.ascontiguousarray(state, dtype=np.uint8)
        out = np.zeros((MAX_LEGAL, MOVE_BYTES), np.uint8)
        n = self._f("legal_moves")(_ptr(s, _u8p), _ptr(out, _u8p))
        return out, int(n)

    def fnn_feature_moves(self, state: np.ndarray):
        s = np.ascontiguousarray(state, dtype=np.uint8)
        out = np.zeros((MAX_LEGAL, MOVE_BYTES), np.uint8)
        n = self._f("fnn_feature_moves")(_ptr(s, _u8p), _ptr(out, _u8p))
        return out, int(n)

    def fnn_features(self, state: np.ndarray, moves: np.ndarray, n: int) -> np.ndarray:
        s = np.ascontiguousarray(state, dtype=np.uint8)
        m = np.zeros((MAX_LEGAL, MOVE_BYTES), np.uint8)
        mv = np.asarray(moves, dtype=np.uint8).reshape(-1, MOVE_BYTES)[:MAX_LEGAL]
        m[: mv.shape[0]] = mv
        f = np.zeros(FEAT_DIM, np.float32)
        self._f("fnn_features")(_ptr(s, _u8p), _ptr(m, _u8p), int(n), _ptr(f, _f32p))
        return f

    def articulation(self, state: np.ndarray) -> np.ndarray:
        s = np.ascontiguousarray(state, dtype=np.uint8)
        out = np.zeros(9, np.uint64)
        self._f("articulation")(_ptr(s, _u8p), _ptr(out, _u64p))
        return out

    def queen_escape(self, state: np.ndarray) -> int:
        s = np.ascontiguousarray(state, dtype=np.uint8)
        return int(self._f("queen_escape")(_ptr(s, _u8p)))


class Oracle(_Engine):
    prefix = "or_"

    def __init__(self, path: str | None = None):
        path = path or os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        lib = ctypes.CDLL(path)
        lib.or_legal_moves.restype = ctypes.c_int
        lib.or_fnn_feature_moves.restype = ctypes.c_int
        lib.or_move_to_action.restype = ctypes.c_int
        lib.or_queen_escape.restype = ctypes.c_int
        lib.or_state_bytes.restype = ctypes.c_int
        lib.or_batch_legal_features_actions.argtypes = [
            _u8p, ctypes.c_int64, _u8p, _i32p, _f32p, _i32p, ctypes.c_int]
        lib.or_batch_successor_features.argtypes = [
            _u8p, _u8p, _i64p, _i64p, ctypes.c_int64, _f32p, ctypes.c_int, ctypes.c_int]
        lib.or_batch_queen_escape.argtypes = [_u8p, ctypes.c_int64, _u8p, ctypes.c_int]
        lib.or_generate_positions.argtypes = [
            ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_uint32, _u8p, _i32p, ctypes.c_int]
        lib.or_lockstep_selfplay.argtypes = lib.or_generate_positions.argtypes
        lib.or_philox4x32_10.argtypes = [ctypes.c_uint32, ctypes.c_uint32, _u32p, _u32p]
        lib.or_batch_root_tactical_probe.argtypes = [
            _u8p, _u8p, _i32p, _f32p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int, _i64p, _u8p, _u8p,
            ctypes.c_int]
        lib.or_surround_count.restype = ctypes.c_int
        lib.or_immediate_win.restype = ctypes.c_int
        super().__init__(lib)
        assert lib.or_state_bytes() == STATE_BYTES

    def centroid(self, state: np.ndarray):
        s = np.ascontiguousarray(state, dtype=np.uint8)
        q, r = ctypes.c_int(), ctypes.c_int()
        self.lib.or_centroid(_ptr(s, _u8p), ctypes.byref(q), ctypes.byref(r))
        return q.value, r.value

    def move_to_action(self, move6, cq: int, cr: int) -> int:
        m = np.ascontiguousarray(np.asarray(move6, dtype=np.uint8).reshape(6))
        return int(self.lib.or_move_to_action(_ptr(m, _u8p), int(cq), int(cr)))

    def neighbor_table(self) -> np.ndarray:
        out = np.zeros((529, 6), np.int16)
        self.lib.or_neighbor_table(_ptr(out, _i16p))
        return out

    def philox(self, key0: int, key1: int, ctr) -> np.ndarray:
        c = np.asarray(ctr, dtype=np.uint32).reshape(4).copy()
        out = np.zeros(4, np.uint32)
        self.lib.or_philox4x32_10(ctypes.c_uint32(key0), ctypes.c_uint32(key1), _ptr(c, _u32p), _ptr(out, _u32p))
        return out

    # batched API ------------------------------------------------------
    def generate_positions(self, B: int, mask: int, max_ply: int, seed: int, threads: int | None = None):
        states = np.zeros((B, STATE_BYTES), np.uint8)
        plies = np.zeros(B, np.int32)
        self.lib.or_generate_positions(B, mask, max_ply, seed, _ptr(states, _u8p), _ptr(plies, _i32p),
                                       threads or default_threads())
        return states, plies

    def lockstep_selfplay(self, G: int, mask: int, max_ply: int, seed: int, threads: int | None = None):
        states = np.zeros((G, STATE_BYTES), np.uint8)
        plies = np.zeros(G, np.int32)
        self.lib.or_lockstep_selfplay(G, mask, max_ply, seed, _ptr(states, _u8p), _ptr(plies, _i32p),
                                      threads or default_threads())
        return states, plies

    def batch_legal_features_actions(self, states: np.ndarray, threads: int | None = None,
                                     want_moves=True, want_features=True, want_actions=True):
        states = np.ascontiguousarray(states, dtype=np.uint8)
        B = states.shape[0]
        moves = np.zeros((B, MAX_LEGAL, MOVE_BYTES), np.uint8) if want_moves else None
        n = np.zeros(B, np.int32)
        feat = np.zeros((B, FEAT_DIM), np.float32) if want_features else None
        act = np.zeros((B, MAX_LEGAL), np.int32) if want_actions else None
        self.lib.or_batch_legal_features_actions(
            _ptr(states, _u8p), B, _ptr(moves, _u8p), _ptr(n, _i32p), _ptr(feat, _f32p), _ptr(act, _i32p),
            threads or default_threads())
        return moves, n, feat, act

    def batch_successor_features(self, states, legal, action_to_root, move_indices, full_list=False,
                                 threads: int | None = None) -> np.ndarray:
        states = np.ascontiguousarray(states, dtype=np.uint8)
        legal = np.ascontiguousarray(legal, dtype=np.uint8)
        a2r = np.ascontiguousarray(action_to_root, dtype=np.int64)
        mi = np.ascontiguousarray(move_indices, dtype=np.int64)
        out = np.zeros((a2r.shape[0], FEAT_DIM), np.float32)
        self.lib.or_batch_successor_features(_ptr(states, _u8p), _ptr(legal, _u8p), _ptr(a2r, _i64p),
                                             _ptr(mi, _i64p), a2r.shape[0], _ptr(out, _f32p),
                                             1 if full_list else 0, threads or default_threads())
        return out

    def batch_queen_escape(self, states, threads: int | None = None) -> np.ndarray:
        states = np.ascontiguousarray(states, dtype=np.uint8)
        out = np.zeros(states.shape[0], np.uint8)
        self.lib.or_batch_queen_escape(_ptr(states, _u8p), states.shape[0], _ptr(out, _u8p),
                                       threads or default_threads())
        return out

    def batch_root_tactical_probe(self, states, legal, num_legal, priors, win1=True, screen=True, win2=True,
                                  threads: int | None = None):
        """(winning [B] int64, allowed [B, 256] uint8, forced [B] uint8) of
        root_tactical_probe_batch (game_logic.cu:290-397)."""
        states = np.ascontiguousarray(states, dtype=np.uint8)
        legal = np.ascontiguousarray(legal, dtype=np.uint8)
        n = np.ascontiguousarray(np.clip(num_legal, -1, MAX_LEGAL), dtype=np.int32)
        pr = np.ascontiguousarray(priors, dtype=np.float32)
        B = states.shape[0]
        win = np.zeros(B, np.int64)
        allowed = np.zeros((B, MAX_LEGAL), np.uint8)
        forced = np.zeros(B, np.uint8)
        self.lib.or_batch_root_tactical_probe(_ptr(states, _u8p), _ptr(legal, _u8p), _ptr(n, _i32p),
                                              _ptr(pr, _f32p), B, int(win1), int(screen), int(win2),
                                              _ptr(win, _i64p), _ptr(allowed, _u8p), _ptr(forced, _u8p),
                                              threads or default_threads())
        return win, allowed, forced

    def cpu_player_search(self, states, weights: dict, num_sims: int, considered: int = 16, c_puct: float = 1.25,
                          c_visit: float = 50.0, c_scale: float = 1.0, threads: int | None = None):
        """FNNNativeCPUPlayer's serial Gumbel search on every state (one game per
        thread, hive_cpu_player.c); weights = the `large` network's state dict as
        float32 numpy arrays.  Returns (chosen slot [G] int32, simulations [G] int64)."""
        states = np.ascontiguousarray(states, dtype=np.uint8)
        G = states.shape[0]
        W = {k: np.ascontiguousarray(v, dtype=np.float32) for k, v in weights.items()}
        fp = ctypes.POINTER(ctypes.c_float)

        class _W(ctypes.Structure):
            _fields_ = [("fc1_w", fp), ("fc1_b", fp), ("ln_w", fp), ("ln_b", fp), ("fc2_w", fp), ("fc2_b", fp),
                        ("value_w", fp), ("value_b", ctypes.c_float), ("a1_w", fp), ("a1_b", fp), ("a2_w", fp),
                        ("a2_b", ctypes.c_float)]

        p = lambda k: W[k].ctypes.data_as(fp)  # noqa: E731
        w = _W(p("fc1.weight"), p("fc1.bias"), p("ln1.weight"), p("ln1.bias"), p("fc2.weight"), p("fc2.bias"),
               p("value_fc.weight"), float(W["value_fc.bias"].reshape(-1)[0]), p("action_fc1.weight"),
               p("action_fc1.bias"), p("action_fc2.weight"), float(W["action_fc2.bias"].reshape(-1)[0]))
        chosen = np.zeros(G, np.int32)
        sims = np.zeros(G, np.int64)
        self.lib.or_cpu_player_search(_ptr(states, _u8p), ctypes.c_int64(G), ctypes.byref(w), int(num_sims),
                                      int(considered), ctypes.c_float(c_puct), ctypes.c_float(c_visit),
                                      ctypes.c_float(c_scale), _ptr(chosen, _i32p), _ptr(sims, _i64p),
                                      int(threads or default_threads()))
        return chosen, sims

    def surround_count(self, state, colour: int) -> int:
        s = np.ascontiguousarray(state, dtype=np.uint8)
        return int(self.lib.or_surround_count(_ptr(s, _u8p), int(colour)))

    def immediate_win(self, state) -> int:
        s = np.ascontiguousarray(state, dtype=np.uint8)
        return int(self.lib.or_immediate_win(_ptr(s, _u8p)))


class Reference(_Engine):
    """The reference's own engine (compiled from /root/reference), or None."""

    prefix = "ref_"

    def __init__(self, lib):
        lib.ref_legal_moves.restype = ctypes.c_int
        lib.ref_fnn_feature_moves.restype = ctypes.c_int
        lib.ref_queen_escape.restype = ctypes.c_int
        lib.ref_state_bytes.restype = ctypes.c_int
        lib.ref_batch_legal_features.argtypes = [_u8p, ctypes.c_int64, _u8p, _i32p, _f32p, ctypes.c_int]
        lib.ref_batch_successor_features.argtypes = [
            _u8p, _u8p, _i64p, _i64p, ctypes.c_int64, _f32p, ctypes.c_int, ctypes.c_int]
        lib.ref_root_tactical_probe.argtypes = [_u8p, _u8p, ctypes.c_int, _f32p, ctypes.c_int, ctypes.c_int,
                                                ctypes.c_int, _i64p, _u8p, _u8p]
        lib.ref_immediate_win.restype = ctypes.c_int
        super().__init__(lib)
        assert lib.ref_state_bytes() == STATE_BYTES
        lib.ref_init()

    @classmethod
    def load(cls):
        path = os.path.join(HERE, "_ref", "libhive_ref.so")
        if not os.path.exists(path):
            return None
        import torch  # noqa: F401  (the shim links libtorch; load it first)
        return cls(ctypes.CDLL(path))

    def batch_legal_features(self, states: np.ndarray, threads: int | None = None):
        states = np.ascontiguousarray(states, dtype=np.uint8)
        B = states.shape[0]
        moves = np.zeros((B, MAX_LEGAL, MOVE_BYTES), np.uint8)
        n = np.zeros(B, np.int32)
        feat = np.zeros((B, FEAT_DIM), np.float32)
        self.lib.ref_batch_legal_features(_ptr(states, _u8p), B, _ptr(moves, _u8p), _ptr(n, _i32p),
                                          _ptr(feat, _f32p), threads or default_threads())
        return moves, n, feat

    def batch_successor_features(self, states, legal, action_to_root, move_indices, full_list=False,
                                 threads: int | None = None) -> np.ndarray:
        states = np.ascontiguousarray(states, dtype=np.uint8)
        legal = np.ascontiguousarray(legal, dtype=np.uint8)
        a2r = np.ascontiguousarray(action_to_root, dtype=np.int64)
        mi = np.ascontiguousarray(move_indices, dtype=np.int64)
        out = np.zeros((a2r.shape[0], FEAT_DIM), np.float32)
        self.lib.ref_batch_successor_features(_ptr(states, _u8p), _ptr(legal, _u8p), _ptr(a2r, _i64p),
                                              _ptr(mi, _i64p), a2r.shape[0], _ptr(out, _f32p),
                                              1 if full_list else 0, threads or default_threads())
        return out

    def root_tactical_probe(self, state, legal, num_legal: int, priors, win1=True, screen=True, win2=True):
        s = np.ascontiguousarray(state, dtype=np.uint8)
        m = np.ascontiguousarray(legal, dtype=np.uint8)
        p = np.ascontiguousarray(priors, dtype=np.float32)
        win = np.zeros(1, np.int64)
        allowed = np.zeros(MAX_LEGAL, np.uint8)
        forced = np.zeros(1, np.uint8)
        self.lib.ref_root_tactical_probe(_ptr(s, _u8p), _ptr(m, _u8p), int(num_legal), _ptr(p, _f32p), int(win1),
                                         int(screen), int(win2), _ptr(win, _i64p), _ptr(allowed, _u8p),
                                         _ptr(forced, _u8p))
        return int(win[0]), allowed, int(forced[0])

    def immediate_win(self, state) -> int:
        s = np.ascontiguousarray(state, dtype=np.uint8)
        return int(self.lib.ref_immediate_win(_ptr(s, _u8p)))
