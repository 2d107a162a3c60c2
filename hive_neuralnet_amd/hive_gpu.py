"""Drop-in counterpart of the reference's ``hive_gpu.load_extension()``.

``load_extension()`` returns an object exposing the reference extension's
entry points (chrismejias/hive_neuralnet hive_gpu/csrc/bindings.cpp:254-476)
with the same names, positional order, keyword defaults, return-tuple order,
dtypes, shapes and fill values, plus its module constants.  Host code is
PyTorch (device memory, the current HIP stream); all compute runs in
``libhive_gpu.so`` through the C-ABI declared in ``include/hive_gpu.h``.

There is no fallback: if the HIP library is missing or the device is not a
GPU, the calls raise.
"""
from __future__ import annotations

import ctypes
import math
import os
import threading

import torch

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libhive_gpu.so")

# constants (bindings.cpp:445-475; state_encoder.cuh:26-46; mcts_tree.cuh:26-27)
BOARD_SIZE = 23
NUM_CELLS = 529
MAX_LEGAL_MOVES = 256
MAX_STACK = 5
SIZEOF_HIVE_STATE = 3424
SIZEOF_GPU_MOVE = 6
OFF_TURN = 3412
OFF_QUEEN_PLACED = 3414
OFF_RESULT = 3415
OFF_STUNNED_CELL = 3416
OFF_QUEEN_CELL = 3392
OFF_HANDS = 3396
OFF_HEIGHT = 2645
ENC_GRID = 17
ACTION_SPACE_SIZE = 85834
PASS_ACTION_INDEX = 85833
MOVEMENT_OFFSET = 2312
DEFAULT_MAX_TREE_NODES = 65536
MAX_TREE_DEPTH = 128
FNN_FEAT_DIM = 122
PROBE_NOALLOC_MAX_ROOTS = 4096  # include/hive_gpu.h HG_PROBE_NOALLOC_MAX_ROOTS
MAX_ENC_NODES = 48
MAX_ENC_EDGES = 200
NODE_FEAT_DIM = 25
EDGE_FEAT_DIM = 9
GLOBAL_FEAT_DIM = 6

_c_void_p = ctypes.c_void_p
_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int

_SIGS = {
    "hg_abi_version": [],
    "hg_initialize_tables": [],
    "hg_create_initial_states": [_c_void_p, _c_i64, _c_int, _c_void_p],
    "hg_apply_moves": [_c_void_p, _c_void_p, _c_i64, _c_void_p],
    "hg_check_results": [_c_void_p, _c_i64, _c_void_p, _c_void_p],
    "hg_generate_legal_moves": [_c_void_p, _c_i64, _c_void_p, _c_void_p, _c_void_p],
    "hg_generate_legal_moves_and_fnn_features": [_c_void_p, _c_i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p],
    "hg_legal_features_actions": [_c_void_p, _c_i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p],
    "hg_legal_features_actions_ordered": [_c_void_p, _c_i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                          _c_int, _c_void_p],
    "hg_extract_fnn_features": [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_void_p, _c_void_p],
    "hg_legal_moves_to_actions": [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_void_p, _c_void_p],
    "hg_compute_centroids": [_c_void_p, _c_i64, _c_void_p, _c_void_p],
    "hg_fnn_successor_features": [_c_void_p, _c_void_p, _c_i64, _c_void_p, _c_void_p, _c_i64, _c_void_p,
                                  _c_void_p],
    "hg_queen_escape_flags": [_c_void_p, _c_i64, _c_void_p, _c_void_p],
    "hg_fnn_leaf_eval": [_c_void_p, _c_i64, _c_i64, ctypes.c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                         _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, ctypes.c_float,
                         _c_void_p, _c_void_p, _c_void_p, ctypes.c_float, _c_void_p, _c_void_p, _c_void_p,
                         _c_void_p, _c_void_p],
    "hg_random_play": [_c_void_p, _c_void_p, _c_i64, _c_int, _c_int, ctypes.c_uint32, _c_void_p, _c_void_p],
    "hg_reserve_candidates": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_int, _c_int, _c_int,
                              _c_void_p, _c_void_p, _c_void_p],
    "hg_candidate_rows": [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_int, _c_int, _c_void_p, _c_void_p],
    "hg_random_play_step": [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_int, _c_int, _c_int, ctypes.c_uint32,
                            _c_void_p, _c_void_p],
    "hg_mcts_select_root_slots": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, ctypes.c_float, _c_i64,
                                  _c_int, _c_int, ctypes.c_float, ctypes.c_float, _c_void_p, _c_void_p, _c_void_p,
                                  _c_void_p, _c_void_p, _c_void_p],
    "hg_mcts_select_root_mask": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, ctypes.c_float, _c_i64, _c_int,
                                 _c_int, ctypes.c_float, ctypes.c_float, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                 _c_void_p, _c_void_p],
    "hg_mcts_replay": [_c_void_p, _c_i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_void_p],
    "hg_mcts_replay_fill": [_c_void_p, _c_i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_void_p],
    "hg_mcts_expand_dense": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                             _c_i64, _c_i64, _c_void_p, _c_void_p],
    "hg_mcts_expand_backprop_dense": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                      _c_void_p, _c_void_p, _c_void_p, _c_void_p, ctypes.c_float, _c_i64, _c_i64,
                                      _c_void_p],
    "hg_mcts_expand_backprop_dense_ws": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                         _c_void_p, _c_void_p, _c_void_p, _c_void_p, ctypes.c_float, _c_i64, _c_i64,
                                         _c_void_p, _c_void_p],
    "hg_mcts_root_noise": [_c_void_p, _c_void_p, _c_void_p, _c_int, ctypes.c_float, ctypes.c_float, _c_i64,
                           _c_void_p],
    "hg_mcts_reset_trees": [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_void_p],
    "hg_mcts_wave_stats": [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_void_p, _c_void_p],
    "hg_gumbel_halving": [_c_void_p, _c_void_p, _c_void_p, _c_int, _c_void_p, ctypes.c_float, ctypes.c_float, _c_int,
                          _c_int, _c_i64, _c_void_p, _c_void_p, _c_void_p],
    "hg_mcts_wave_root_slots": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, ctypes.c_float,
                                _c_i64, _c_int, _c_int, ctypes.c_float, ctypes.c_float, _c_void_p, _c_void_p,
                                _c_void_p],
    "hg_legal_mask": [_c_void_p, _c_i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p],
    "hg_mcts_select": [_c_void_p, _c_void_p, _c_void_p, ctypes.c_float, _c_i64, _c_int, _c_void_p, _c_void_p,
                       _c_void_p, _c_void_p, _c_void_p, _c_void_p],
    "hg_mcts_expand": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64,
                       _c_void_p, _c_void_p],
    "hg_mcts_backprop": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_void_p],
    "hg_mcts_expand_backprop": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_void_p],
    "hg_mcts_extract_policy": [_c_void_p, _c_void_p, _c_void_p, ctypes.c_float, _c_int, ctypes.c_float, _c_i64,
                               _c_void_p, _c_void_p],
    "hg_successor_rows": [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_void_p, _c_void_p, _c_void_p],
    "hg_fnn_leaf_eval_lists": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_int, _c_void_p, _c_void_p,
                               _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, ctypes.c_float, _c_void_p,
                               _c_void_p, _c_void_p, ctypes.c_float, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                               _c_void_p],
    "hg_root_tactical_probe": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_int, _c_int, _c_int, _c_void_p,
                               _c_void_p, _c_void_p, _c_void_p, _c_void_p],
    "hg_probe_scratch_init": [],
    "hg_root_tactical_probe_noalloc": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_int, _c_int, _c_int,
                                       _c_void_p, _c_void_p, _c_void_p, _c_void_p],
}
_SIGS_I64 = {  # entry points returning a size (int64_t)
    "hg_root_tactical_probe_workspace": [_c_i64],
    "hg_successor_rows_workspace": [_c_i64],
    "hg_fnn_leaf_eval_lists_workspace": [_c_i64, _c_int],
    "hg_mcts_expand_backprop_dense_workspace": [_c_i64, _c_i64],
    "hg_legal_features_actions_ordered_workspace": [_c_i64],
}


class HgTree(ctypes.Structure):
    """C layout of `hg_tree` (include/hive_gpu.h)."""

    _fields_ = [(name, ctypes.c_void_p) for name in (
        "visit_count", "total_value", "prior", "parent_idx", "virtual_q_penalty", "move_bytes", "action_idx",
        "first_child", "num_children", "is_terminal", "terminal_value", "node_count", "child_init_q")] + [
        ("max_nodes", ctypes.c_int64)]


class HgFnnNet(ctypes.Structure):
    """C layout of `hg_fnn_net` (include/hive_gpu.h)."""

    _fields_ = [(name, ctypes.c_void_p) for name in (
        "fc1_w", "fc1_b", "ln_w", "ln_b", "fc2_w", "fc2_b", "value_w", "action1_w", "action1_b", "action2_w")] + [
        ("value_b", ctypes.c_float), ("action2_b", ctypes.c_float), ("F", ctypes.c_int32)]


class HgWaveBuffers(ctypes.Structure):
    """C layout of `hg_wave_buffers` (include/hive_gpu.h)."""

    _fields_ = [(name, ctypes.c_void_p) for name in (
        "leaf_idx", "move_paths", "path_lens", "vl_paths", "vl_lens", "leaf_states", "results", "legal_moves",
        "num_legal", "features", "priors", "values", "child_q", "leaf_workspace", "tree_workspace", "stats")] + [
        ("capacity", ctypes.c_int64)]


_TREE_SPEC = [  # the 12 tree tensors in the reference's argument order (game_logic.cu:933-953)
    ("vc", torch.int32), ("tv", torch.float32), ("pr", torch.float32), ("pa", torch.int32),
    ("vq", torch.float32), ("mb", torch.uint8), ("ai", torch.int32), ("fc", torch.int32),
    ("nc", torch.int32), ("it", torch.int8), ("tv2", torch.float32), ("cnt", torch.int32),
]


def _tree_struct(tensors, child_init_q, B: int, max_nodes: int) -> HgTree:
    """Validate the 12 tree tensors + child_init_q and pack their pointers."""
    if len(tensors) != 12:
        raise ValueError("expected the 12 tree tensors")
    ptrs = []
    for (name, dtype), t in zip(_TREE_SPEC, tensors):
        if name == "mb":
            _dev(t, name, dtype, (max_nodes, SIZEOF_GPU_MOVE), B)
        elif name == "cnt":
            _dev(t, name, dtype, (), B)
        else:
            _dev(t, name, dtype, (max_nodes,), B)
        ptrs.append(t.data_ptr())
    _dev(child_init_q, "child_init_q", torch.float32, (max_nodes,), B)
    vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt = ptrs
    return HgTree(vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt, child_init_q.data_ptr(), int(max_nodes))


def _select_outputs(T: int, whole_rows: bool = False):
    """Select outputs; zero-filled unless the kernel writes whole rows."""
    new = torch.empty if whole_rows else torch.zeros
    leaf = new((T,), dtype=torch.int32, device="cuda")
    paths = new((T, MAX_TREE_DEPTH, SIZEOF_GPU_MOVE), dtype=torch.uint8, device="cuda")
    plen = new((T,), dtype=torch.int32, device="cuda")
    vl = new((T, MAX_TREE_DEPTH), dtype=torch.int32, device="cuda")
    vlen = new((T,), dtype=torch.int32, device="cuda")
    return leaf, paths, plen, vl, vlen

_lib = None
_lib_lock = threading.Lock()
# root_tactical_probe_batch_noalloc: per device, an event recorded after the
# last call (the next call's stream waits on it: the calls share the scratch)
_noalloc_lock = threading.Lock()
_noalloc_done: dict = {}


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libhive_gpu.so and declare its C-ABI; raises if it is not built."""
    global _lib
    with _lib_lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise RuntimeError(
                f"{path} is missing: build the HIP engine with `python -m hive_neuralnet_amd.build`")
        lib = ctypes.CDLL(path)
        for name, args in _SIGS.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        for name, args in _SIGS_I64.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = _c_i64
        _lib = lib
        return lib


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _check(err: int, what: str) -> None:
    if err != 0:
        raise RuntimeError(f"{what}: HIP error {err}")


def _dev(t: torch.Tensor, name: str, dtype: torch.dtype, inner: tuple, rows: int) -> torch.Tensor:
    """Validate a device tensor: dtype, trailing shape, >= rows rows, contiguous.

    A tensor whose trailing shape differs is accepted only when it is flat
    (1-D) and contiguous, as a view of rows of `inner` (never a copy: an
    output buffer the kernel writes must be the caller's memory)."""
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if inner and tuple(t.shape[-len(inner):]) != tuple(inner):
        size = math.prod(inner)
        if t.dim() == 1 and t.is_contiguous() and t.numel() % size == 0:
            t = t.view(-1, *inner)
        else:
            raise ValueError(f"{name} must have trailing shape {inner}, got {tuple(t.shape)}")
    lead = t.shape[0] if t.dim() > len(inner) else 1
    if lead < rows:
        raise ValueError(f"{name} has {lead} rows, need {rows}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t


def _state_rows(states: torch.Tensor, rows: int) -> torch.Tensor:
    return _dev(states, "states", torch.uint8, (SIZEOF_HIVE_STATE,), rows)


class HiveGpuExtension:
    """The reference extension's Python surface on top of libhive_gpu.so."""

    def __init__(self, lib: ctypes.CDLL):
        self._lib = lib
        # turn-ordered legal lists: per (device, stream) a zero-filled workspace
        # kept across calls and the parity of its next call
        self._order_ws = {}
        self._order_lock = threading.Lock()
        for k, v in globals().items():
            if k.isupper() and isinstance(v, int):
                setattr(self, k, v)

    # ---- tables / state tensors -------------------------------------------
    def initialize_tables(self) -> None:
        _check(self._lib.hg_initialize_tables(), "initialize_tables")

    def create_initial_states(self, batch_size: int, expansion_mask: int = 0) -> torch.Tensor:
        B = int(batch_size)
        states = torch.empty((B, SIZEOF_HIVE_STATE), dtype=torch.uint8, device="cuda")
        _check(self._lib.hg_create_initial_states(states.data_ptr(), B, int(expansion_mask), _stream()),
               "create_initial_states")
        return states

    def apply_moves_batch(self, states: torch.Tensor, moves: torch.Tensor, batch_size: int) -> None:
        B = int(batch_size)
        states = _state_rows(states, B)
        moves = _dev(moves, "moves", torch.uint8, (SIZEOF_GPU_MOVE,), B)
        _check(self._lib.hg_apply_moves(states.data_ptr(), moves.data_ptr(), B, _stream()), "apply_moves_batch")

    def check_results_batch(self, states: torch.Tensor, batch_size: int) -> torch.Tensor:
        B = int(batch_size)
        states = _state_rows(states, B)
        out = torch.empty((B,), dtype=torch.int32, device="cuda")
        _check(self._lib.hg_check_results(states.data_ptr(), B, out.data_ptr(), _stream()), "check_results_batch")
        return out

    # ---- move generation / features / actions -----------------------------
    def generate_legal_moves_batch(self, states: torch.Tensor, batch_size: int):
        B = int(batch_size)
        states = _state_rows(states, B)
        moves = torch.empty((B, MAX_LEGAL_MOVES, SIZEOF_GPU_MOVE), dtype=torch.uint8, device="cuda")
        n = torch.empty((B,), dtype=torch.int32, device="cuda")
        _check(self._lib.hg_generate_legal_moves(states.data_ptr(), B, moves.data_ptr(), n.data_ptr(), _stream()),
               "generate_legal_moves_batch")
        return moves, n

    def generate_legal_moves_and_fnn_features_batch(self, states: torch.Tensor, batch_size: int):
        B = int(batch_size)
        states = _state_rows(states, B)
        moves = torch.empty((B, MAX_LEGAL_MOVES, SIZEOF_GPU_MOVE), dtype=torch.uint8, device="cuda")
        n = torch.empty((B,), dtype=torch.int32, device="cuda")
        feat = torch.empty((B, FNN_FEAT_DIM), dtype=torch.float32, device="cuda")
        _check(self._lib.hg_generate_legal_moves_and_fnn_features(
            states.data_ptr(), B, moves.data_ptr(), n.data_ptr(), feat.data_ptr(), _stream()),
            "generate_legal_moves_and_fnn_features_batch")
        return moves, n, feat

    def generate_legal_moves_features_actions_batch(self, states: torch.Tensor, batch_size: int,
                                                    ordered: bool = True):
        """Fused: (moves, num_legal, features, action_indices) in one pass.  With
        `ordered` (default) the positions are taken in buckets of turns, latest
        first (hg_legal_features_actions_ordered): the same outputs, a shorter
        launch on batches of mixed game stages.  Its int32 workspace is kept per
        (device, stream) and its two count arrays are used in turn, so a call
        made while the stream is being captured into a HIP graph (whose replays
        would all repeat the captured turn) takes the index order instead."""
        B = int(batch_size)
        states = _state_rows(states, B)
        moves = torch.empty((B, MAX_LEGAL_MOVES, SIZEOF_GPU_MOVE), dtype=torch.uint8, device="cuda")
        n = torch.empty((B,), dtype=torch.int32, device="cuda")
        feat = torch.empty((B, FNN_FEAT_DIM), dtype=torch.float32, device="cuda")
        act = torch.empty((B, MAX_LEGAL_MOVES), dtype=torch.int32, device="cuda")
        if ordered and B > 0 and not torch.cuda.is_current_stream_capturing():
            stream = _stream()
            key = (torch.cuda.current_device(), stream)
            need = int(self._lib.hg_legal_features_actions_ordered_workspace(B)) // 4
            with self._order_lock:
                ws, parity = self._order_ws.get(key, (None, 0))
                if ws is None or ws.numel() < need:
                    ws, parity = torch.zeros((need,), dtype=torch.int32, device="cuda"), 0
                # dropped while the call is in flight, so a failed call leaves no half-used workspace
                self._order_ws.pop(key, None)
            _check(self._lib.hg_legal_features_actions_ordered(
                states.data_ptr(), B, moves.data_ptr(), n.data_ptr(), feat.data_ptr(), act.data_ptr(),
                ws.data_ptr(), parity, stream), "generate_legal_moves_features_actions_batch")
            with self._order_lock:
                self._order_ws[key] = (ws, parity ^ 1)
        else:
            _check(self._lib.hg_legal_features_actions(
                states.data_ptr(), B, moves.data_ptr(), n.data_ptr(), feat.data_ptr(), act.data_ptr(), _stream()),
                "generate_legal_moves_features_actions_batch")
        return moves, n, feat, act

    def extract_fnn_features_batch(self, states, legal_moves, num_legal, batch_size: int) -> torch.Tensor:
        B = int(batch_size)
        states = _state_rows(states, B)
        legal_moves = _dev(legal_moves, "legal_moves", torch.uint8, (MAX_LEGAL_MOVES, SIZEOF_GPU_MOVE), B)
        num_legal = _dev(num_legal, "num_legal", torch.int32, (), B)
        feat = torch.empty((B, FNN_FEAT_DIM), dtype=torch.float32, device="cuda")
        _check(self._lib.hg_extract_fnn_features(states.data_ptr(), legal_moves.data_ptr(), num_legal.data_ptr(), B,
                                                 feat.data_ptr(), _stream()), "extract_fnn_features_batch")
        return feat

    def legal_moves_to_actions_batch(self, states, legal_moves, num_legal, batch_size: int) -> torch.Tensor:
        B = int(batch_size)
        states = _state_rows(states, B)
        legal_moves = _dev(legal_moves, "legal_moves", torch.uint8, (MAX_LEGAL_MOVES, SIZEOF_GPU_MOVE), B)
        num_legal = _dev(num_legal, "num_legal", torch.int32, (), B)
        act = torch.empty((B, MAX_LEGAL_MOVES), dtype=torch.int32, device="cuda")
        _check(self._lib.hg_legal_moves_to_actions(states.data_ptr(), legal_moves.data_ptr(), num_legal.data_ptr(),
                                                   B, act.data_ptr(), _stream()), "legal_moves_to_actions_batch")
        return act

    def compute_centroids_batch(self, states: torch.Tensor, batch_size: int) -> torch.Tensor:
        B = int(batch_size)
        states = _state_rows(states, B)
        out = torch.empty((B, 2), dtype=torch.int32, device="cuda")
        _check(self._lib.hg_compute_centroids(states.data_ptr(), B, out.data_ptr(), _stream()),
               "compute_centroids_batch")
        torch.cuda.current_stream().synchronize()  # the reference synchronises here (game_logic.cu:923)
        return out

    def fnn_successor_features_batch(self, states, legal_moves, action_to_root, move_indices,
                                     num_actions: int, out: torch.Tensor | None = None) -> torch.Tensor:
        """`out` (extension): an existing [N, 122] float32 buffer to write into."""
        N = int(num_actions)
        states = _dev(states, "states", torch.uint8, (SIZEOF_HIVE_STATE,), 0)
        legal_moves = _dev(legal_moves, "legal_moves", torch.uint8, (MAX_LEGAL_MOVES, SIZEOF_GPU_MOVE), 0)
        action_to_root = _dev(action_to_root, "action_to_root", torch.int64, (), N)
        move_indices = _dev(move_indices, "move_indices", torch.int64, (), N)
        if out is None:
            feat = torch.empty((N, FNN_FEAT_DIM), dtype=torch.float32, device="cuda")
        else:
            feat = _dev(out, "out", torch.float32, (FNN_FEAT_DIM,), N)
        roots = min(states.numel() // SIZEOF_HIVE_STATE, legal_moves.numel() // (MAX_LEGAL_MOVES * SIZEOF_GPU_MOVE))
        _check(self._lib.hg_fnn_successor_features(states.data_ptr(), legal_moves.data_ptr(), roots,
                                                   action_to_root.data_ptr(), move_indices.data_ptr(), N,
                                                   feat.data_ptr(), _stream()), "fnn_successor_features_batch")
        return feat

    # ---- fused FNN leaf evaluation (no reference counterpart; see include/hive_gpu.h)
    def fnn_leaf_eval(self, features, T: int, offsets, num_legal, succ_leaf, net, head_biases=None):
        """(priors [T, 256], leaf values [T], child Q [T, 256]) from the feature
        rows [T + N, F] (leaf rows, then successor rows grouped by leaf) through
        the 64-wide HiveFNN `net` (fc1, ln1, fc2, value_fc, action_fc1, action_fc2).
        `head_biases` = (value_fc.bias, action_fc2.bias) as floats, when the
        caller already holds them on the host (saves two device reads)."""
        T = int(T)
        F = features.shape[1]
        N = features.shape[0] - T
        features = _dev(features, "features", torch.float32, (F,), T + N)
        offsets = _dev(offsets, "offsets", torch.int64, (), T)
        num_legal = _dev(num_legal, "num_legal", torch.int32, (), T)
        succ_leaf = _dev(succ_leaf, "succ_leaf", torch.int64, (), N)
        w, vb, ab = _fnn_weights(net, F, head_biases)
        ws = torch.empty((T * 64 + 2 * N,), dtype=torch.float32, device="cuda")
        priors = torch.empty((T, MAX_LEGAL_MOVES), dtype=torch.float32, device="cuda")
        child_q = torch.empty((T, MAX_LEGAL_MOVES), dtype=torch.float32, device="cuda")
        values = torch.empty((T,), dtype=torch.float32, device="cuda")
        _check(self._lib.hg_fnn_leaf_eval(
            features.data_ptr(), T, N, F, offsets.data_ptr(), num_legal.data_ptr(), succ_leaf.data_ptr(),
            w[0].data_ptr(), w[1].data_ptr(), w[2].data_ptr(), w[3].data_ptr(), w[4].data_ptr(), w[5].data_ptr(),
            w[6].data_ptr(), vb, w[7].data_ptr(), w[8].data_ptr(), w[9].data_ptr(), ab, ws.data_ptr(),
            priors.data_ptr(), values.data_ptr(), child_q.data_ptr(), _stream()), "fnn_leaf_eval")
        return priors, values, child_q

    def fnn_leaf_eval_lists(self, leaf_states, legal_moves, num_legal, root_features, T: int, net,
                            head_biases=None, workspace: torch.Tensor | None = None):
        """(priors [T, 256], leaf values [T], child Q [T, 256]) of the leaves
        from their own legal lists, with no host synchronisation: successor
        rows sized on the device (hg_fnn_leaf_eval_lists).  `workspace`: a
        uint8 device buffer of at least workspace_bytes(T) to reuse."""
        T = int(T)
        F = FNN_FEAT_DIM
        leaf_states = _state_rows(leaf_states, T)
        legal_moves = _dev(legal_moves, "legal_moves", torch.uint8, (MAX_LEGAL_MOVES, SIZEOF_GPU_MOVE), T)
        num_legal = _dev(num_legal, "num_legal", torch.int32, (), T)
        root_features = _dev(root_features, "root_features", torch.float32, (F,), T)
        w, vb, ab = _fnn_weights(net, F, head_biases)
        need = int(self._lib.hg_fnn_leaf_eval_lists_workspace(T, F))
        if workspace is None or workspace.numel() < need + 256:
            workspace = torch.empty((need + 256,), dtype=torch.uint8, device="cuda")
        ptr = (workspace.data_ptr() + 255) & ~255
        priors = torch.empty((T, MAX_LEGAL_MOVES), dtype=torch.float32, device="cuda")
        child_q = torch.empty((T, MAX_LEGAL_MOVES), dtype=torch.float32, device="cuda")
        values = torch.empty((T,), dtype=torch.float32, device="cuda")
        if T > 0:
            _check(self._lib.hg_fnn_leaf_eval_lists(
                leaf_states.data_ptr(), legal_moves.data_ptr(), num_legal.data_ptr(), root_features.data_ptr(), T, F,
                w[0].data_ptr(), w[1].data_ptr(), w[2].data_ptr(), w[3].data_ptr(), w[4].data_ptr(),
                w[5].data_ptr(), w[6].data_ptr(), vb, w[7].data_ptr(), w[8].data_ptr(), w[9].data_ptr(), ab, ptr,
                priors.data_ptr(), values.data_ptr(), child_q.data_ptr(), _stream()), "fnn_leaf_eval_lists")
        return priors, values, child_q

    def tree_struct(self, vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt, child_init_q, B: int,
                    max_nodes: int) -> HgTree:
        """The 12 tree tensors + child_init_q validated and packed once (an
        `hg_tree` to pass by reference to the entry points that take one)."""
        return _tree_struct((vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt), child_init_q, int(B), int(max_nodes))

    def gumbel_halving(self, tree: HgTree, root_nodes, candidates, base, c_visit: float, c_scale: float,
                       root_q_min_visits: int, final: bool = False):
        """One sequential-halving decision (hg_gumbel_halving) over a packed
        tree: the next round's candidates [B, C // 2] int32, or with `final`
        the chosen slot [B] int64.  candidates [B, C] int32 (C <= 64), base
        [B, 256] f32 (Gumbel + legal logits)."""
        if candidates.dim() != 2:
            raise ValueError("candidates must be [B, C]")
        B, C = int(candidates.shape[0]), int(candidates.shape[1])
        _dev(candidates, "candidates", torch.int32, (C,), B)
        _dev(root_nodes, "root_nodes", torch.int32, (), B)
        _dev(base, "base", torch.float32, (MAX_LEGAL_MOVES,), B)
        keep = 0 if final else C // 2
        if final:
            out = torch.empty((B,), dtype=torch.int64, device="cuda")
            args = (None, out.data_ptr())
        else:
            out = torch.empty((B, keep), dtype=torch.int32, device="cuda")
            args = (out.data_ptr(), None)
        if keep == 0 and not final:
            return out
        _check(self._lib.hg_gumbel_halving(ctypes.byref(tree), root_nodes.data_ptr(), candidates.data_ptr(), C,
                                           base.data_ptr(), float(c_visit), float(c_scale), int(root_q_min_visits),
                                           keep, B, *args, _stream()), "gumbel_halving")
        return out

    def prepare_wave_root_slots(self, vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt, child_init_q, B: int,
                                max_nodes: int, net, head_biases=None, capacity: int | None = None) -> "WavePlan":
        """A WavePlan: simulation waves of the Gumbel root search over this
        tree and network (hg_mcts_wave_root_slots), for up to `capacity`
        simulations per wave (default 16 * B)."""
        return WavePlan(self._lib, (vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt), child_init_q, B, max_nodes,
                        net, head_biases, capacity if capacity is not None else 16 * int(B))

    def leaf_eval_workspace_bytes(self, T: int) -> int:
        return int(self._lib.hg_fnn_leaf_eval_lists_workspace(int(T), FNN_FEAT_DIM)) + 256

    def root_tactical_probe_batch(self, states, legal_moves, num_legal, priors, batch_size: int,
                                  enable_win_in_one: bool = True, enable_check_opponent_wins: bool = True,
                                  enable_win_in_two: bool = True):
        """(winning [B] int64, -1 filled; allowed [B, 256] uint8; forced [B] uint8)
        -- bindings.cpp:336-344 / game_logic.cu:1579-1616."""
        B = int(batch_size)
        if B <= 0:
            return (torch.full((0,), -1, dtype=torch.int64, device="cuda"),
                    torch.zeros((0, MAX_LEGAL_MOVES), dtype=torch.uint8, device="cuda"),
                    torch.zeros((0,), dtype=torch.uint8, device="cuda"))
        states = _state_rows(states, B)
        legal_moves = _dev(legal_moves, "legal_moves", torch.uint8, (MAX_LEGAL_MOVES, SIZEOF_GPU_MOVE), B)
        num_legal = _dev(num_legal, "num_legal", torch.int32, (), B)
        priors = _dev(priors, "priors", torch.float32, (MAX_LEGAL_MOVES,), B)
        winning = torch.empty((B,), dtype=torch.int64, device="cuda")
        allowed = torch.empty((B, MAX_LEGAL_MOVES), dtype=torch.uint8, device="cuda")
        forced = torch.empty((B,), dtype=torch.uint8, device="cuda")
        ws = torch.empty((int(self._lib.hg_root_tactical_probe_workspace(B)),), dtype=torch.int32, device="cuda")
        _check(self._lib.hg_root_tactical_probe(states.data_ptr(), legal_moves.data_ptr(), num_legal.data_ptr(),
                                                priors.data_ptr(), B, int(bool(enable_win_in_one)),
                                                int(bool(enable_check_opponent_wins)), int(bool(enable_win_in_two)),
                                                winning.data_ptr(), allowed.data_ptr(), forced.data_ptr(),
                                                ws.data_ptr(), _stream()), "root_tactical_probe_batch")
        return winning, allowed, forced

    def root_tactical_probe_batch_noalloc(self, states, legal_moves, num_legal, priors, batch_size: int,
                                          enable_win_in_one: bool = True, enable_check_opponent_wins: bool = True,
                                          enable_win_in_two: bool = True, out=None):
        """root_tactical_probe_batch without a device allocation in the call
        (extension; hg_root_tactical_probe_noalloc): the job lists live in the
        library's per-GPU scratch array, for at most PROBE_NOALLOC_MAX_ROOTS
        roots.  `out` = (winning [B] int64, allowed [B, 256] uint8, forced [B]
        uint8) buffers to write; when None they are allocated here.  Calls
        on one GPU share the scratch: this method orders its own calls on a
        device (each waits on an event recorded after the previous one, on
        whichever stream), except under graph capture, where overlapping
        replays are the caller's to serialise."""
        B = int(batch_size)
        if B > PROBE_NOALLOC_MAX_ROOTS:
            raise ValueError(f"root_tactical_probe_batch_noalloc: {B} roots, at most {PROBE_NOALLOC_MAX_ROOTS}")
        if out is None:
            out = (torch.empty((max(B, 0),), dtype=torch.int64, device="cuda"),
                   torch.empty((max(B, 0), MAX_LEGAL_MOVES), dtype=torch.uint8, device="cuda"),
                   torch.empty((max(B, 0),), dtype=torch.uint8, device="cuda"))
        winning = _dev(out[0], "winning", torch.int64, (), B)
        allowed = _dev(out[1], "allowed", torch.uint8, (MAX_LEGAL_MOVES,), B)
        forced = _dev(out[2], "forced", torch.uint8, (), B)
        if B <= 0:
            return winning, allowed, forced
        states = _state_rows(states, B)
        legal_moves = _dev(legal_moves, "legal_moves", torch.uint8, (MAX_LEGAL_MOVES, SIZEOF_GPU_MOVE), B)
        num_legal = _dev(num_legal, "num_legal", torch.int32, (), B)
        priors = _dev(priors, "priors", torch.float32, (MAX_LEGAL_MOVES,), B)
        capturing = torch.cuda.is_current_stream_capturing()
        with _noalloc_lock:
            dev = torch.cuda.current_device()
            done = _noalloc_done.get(dev)
            if done is not None and not capturing:
                torch.cuda.current_stream().wait_event(done)
            _check(self._lib.hg_root_tactical_probe_noalloc(
                states.data_ptr(), legal_moves.data_ptr(), num_legal.data_ptr(), priors.data_ptr(), B,
                int(bool(enable_win_in_one)), int(bool(enable_check_opponent_wins)), int(bool(enable_win_in_two)),
                winning.data_ptr(), allowed.data_ptr(), forced.data_ptr(), _stream()),
                "root_tactical_probe_batch_noalloc")
            if not capturing:
                if done is None:
                    done = _noalloc_done[dev] = torch.cuda.Event()
                done.record()
        return winning, allowed, forced

    def generate_legal_mask_batch(self, states: torch.Tensor, batch_size: int):
        """(masks [B, 85834] f32, num_legal [B] i32) -- bindings.cpp:292-294."""
        moves, n, masks = self.generate_legal_moves_and_mask_batch(states, batch_size)
        return masks, n

    def generate_legal_moves_and_mask_batch(self, states: torch.Tensor, batch_size: int):
        """(moves [B, 256, 6] u8, num_legal [B] i32, masks [B, 85834] f32) -- bindings.cpp:296-298."""
        B = int(batch_size)
        states = _state_rows(states, B)
        moves = torch.empty((B, MAX_LEGAL_MOVES, SIZEOF_GPU_MOVE), dtype=torch.uint8, device="cuda")
        n = torch.empty((B,), dtype=torch.int32, device="cuda")
        masks = torch.empty((B, ACTION_SPACE_SIZE), dtype=torch.float32, device="cuda")
        acts = torch.empty((B, MAX_LEGAL_MOVES), dtype=torch.int32, device="cuda")
        _check(self._lib.hg_legal_mask(states.data_ptr(), B, moves.data_ptr(), n.data_ptr(), acts.data_ptr(),
                                       masks.data_ptr(), _stream()), "generate_legal_moves_and_mask_batch")
        return moves, n, masks

    def reserve_candidates(self, states, legal_moves, num_legal, batch_size: int, immobile_only: bool = True,
                           priors=None, k: int = 16, reserve: int = 6, allowed=None, want_qualifies: bool = True):
        """Reserve-slot qualification and, with priors, the Gumbel root candidate
        rows in one launch (hg_reserve_candidates; FNNMCTSOrchestrator.
        _root_candidate_slots with reserve slots, fnn_mcts_orchestrator.py:338-444).
        Returns (qualifies [B, 256] bool or None, candidates [B, k] int32 or None)."""
        B = int(batch_size)
        states = _state_rows(states, B)
        legal_moves = _dev(legal_moves, "legal_moves", torch.uint8, (MAX_LEGAL_MOVES, SIZEOF_GPU_MOVE), B)
        num_legal = _dev(num_legal, "num_legal", torch.int32, (), B)
        qual = torch.empty((B, MAX_LEGAL_MOVES), dtype=torch.uint8, device="cuda") if want_qualifies else None
        cand = None
        if priors is not None:
            priors = _dev(priors, "priors", torch.float32, (MAX_LEGAL_MOVES,), B)
            cand = torch.empty((B, int(k)), dtype=torch.int32, device="cuda")
        if allowed is not None:
            allowed = _dev(allowed.to(torch.uint8).contiguous(), "allowed", torch.uint8, (MAX_LEGAL_MOVES,), B)
        _check(self._lib.hg_reserve_candidates(
            states.data_ptr(), legal_moves.data_ptr(), num_legal.data_ptr(),
            allowed.data_ptr() if allowed is not None else None, priors.data_ptr() if priors is not None else None,
            B, int(k), int(reserve), 1 if immobile_only else 0, qual.data_ptr() if qual is not None else None,
            cand.data_ptr() if cand is not None else None, _stream()), "reserve_candidates")
        return (qual.to(torch.bool) if qual is not None else None), cand

    def candidate_rows(self, qualifies, valid, priors, k: int, reserve: int) -> torch.Tensor:
        """The candidate rows of reserve_candidates from given [B, 256] masks (hg_candidate_rows)."""
        B = int(priors.shape[0])
        q = _dev(qualifies.to(torch.uint8).contiguous(), "qualifies", torch.uint8, (MAX_LEGAL_MOVES,), B)
        v = _dev(valid.to(torch.uint8).contiguous(), "valid", torch.uint8, (MAX_LEGAL_MOVES,), B)
        priors = _dev(priors, "priors", torch.float32, (MAX_LEGAL_MOVES,), B)
        cand = torch.empty((B, int(k)), dtype=torch.int32, device="cuda")
        _check(self._lib.hg_candidate_rows(q.data_ptr(), v.data_ptr(), priors.data_ptr(), B, int(k), int(reserve),
                                           cand.data_ptr(), _stream()), "candidate_rows")
        return cand

    def queen_escape_flags_batch(self, states: torch.Tensor, batch_size: int) -> torch.Tensor:
        B = int(batch_size)
        states = _state_rows(states, B)
        out = torch.empty((B,), dtype=torch.uint8, device="cuda")
        _check(self._lib.hg_queen_escape_flags(states.data_ptr(), B, out.data_ptr(), _stream()),
               "queen_escape_flags_batch")
        return out


def _fnn_weights(net, F: int, head_biases=None):
    """The ten weight tensors of a 64-wide HiveFNN as flat device float32
    arrays, and the two head biases as host floats."""
    spec = ((net.fc1.weight, "fc1.weight", 64 * F), (net.fc1.bias, "fc1.bias", 64),
            (net.ln1.weight, "ln1.weight", 64), (net.ln1.bias, "ln1.bias", 64),
            (net.fc2.weight, "fc2.weight", 64 * 64), (net.fc2.bias, "fc2.bias", 64),
            (net.value_fc.weight, "value_fc.weight", 64), (net.action_fc1.weight, "action_fc1.weight", 64 * 128),
            (net.action_fc1.bias, "action_fc1.bias", 64), (net.action_fc2.weight, "action_fc2.weight", 64))
    w = []
    for t, name, n in spec:
        if t.numel() != n:
            raise ValueError(f"fnn_leaf_eval serves 64-wide networks: {name} has {t.numel()} values, need {n}")
        w.append(_dev(t.detach().reshape(-1), name, torch.float32, (), n))
    if head_biases is None:
        head_biases = (net.value_fc.bias.detach().reshape(-1)[0].item(),
                       net.action_fc2.bias.detach().reshape(-1)[0].item())
    return w, float(head_biases[0]), float(head_biases[1])


class WavePlan:
    """hg_mcts_wave_root_slots with its fixed arguments prepared once.

    The tree (12 arrays + child_init_q) and the 64-wide network are validated
    and packed here, and the per-simulation buffers are allocated for
    `capacity` simulations; each run() then costs one library call.  The
    tensors stay referenced by the plan, so their addresses stay valid;
    the network enters by address (weights updated in place are seen, a
    re-created network needs a new plan).  run() returns views of the
    plan's buffers, which the next run() overwrites in stream order."""

    def __init__(self, lib, tree_tensors, child_init_q, B: int, max_nodes: int, net, head_biases, capacity: int):
        B, M, cap = int(B), int(max_nodes), int(capacity)
        if B <= 0 or cap <= 0:
            raise ValueError("WavePlan: B and capacity must be positive")
        self._lib = lib
        self.B, self.max_nodes, self.capacity = B, M, cap
        self._keep = (tuple(tree_tensors), child_init_q)
        self._tree = _tree_struct(tuple(tree_tensors), child_init_q, B, M)
        self.set_net(net, head_biases)

        def buf(shape, dtype):
            return torch.empty(shape, dtype=dtype, device="cuda")

        self.leaf_idx = buf((cap,), torch.int32)
        self.move_paths = buf((cap, MAX_TREE_DEPTH, SIZEOF_GPU_MOVE), torch.uint8)
        self.path_lens = buf((cap,), torch.int32)
        self.vl_paths = buf((cap, MAX_TREE_DEPTH), torch.int32)
        self.vl_lens = buf((cap,), torch.int32)
        self.leaf_states = buf((cap, SIZEOF_HIVE_STATE), torch.uint8)
        self.results = buf((cap,), torch.int32)
        self.legal_moves = buf((cap, MAX_LEGAL_MOVES, SIZEOF_GPU_MOVE), torch.uint8)
        self.num_legal = buf((cap,), torch.int32)
        self.features = buf((cap, FNN_FEAT_DIM), torch.float32)
        self.priors = buf((cap, MAX_LEGAL_MOVES), torch.float32)
        self.values = buf((cap,), torch.float32)
        self.child_q = buf((cap, MAX_LEGAL_MOVES), torch.float32)
        # both workspaces grow with the simulation count: sized at capacity they
        # serve every smaller wave
        self._leaf_ws = buf((int(lib.hg_fnn_leaf_eval_lists_workspace(cap, FNN_FEAT_DIM)) + 256,), torch.uint8)
        self._tree_ws = buf((max(1, (int(lib.hg_mcts_expand_backprop_dense_workspace(B, cap)) + 3) // 4),),
                            torch.int32)
        ptrs = [t.data_ptr() for t in (self.leaf_idx, self.move_paths, self.path_lens, self.vl_paths, self.vl_lens,
                                       self.leaf_states, self.results, self.legal_moves, self.num_legal,
                                       self.features, self.priors, self.values, self.child_q)]
        self._bufs = HgWaveBuffers(*ptrs, (self._leaf_ws.data_ptr() + 255) & ~255, self._tree_ws.data_ptr(), None,
                                   cap)

    def tree_base(self) -> int:
        """Address of the plan's visit_count array (its first game's row)."""
        return self._keep[0][0].data_ptr()

    def set_net(self, net, head_biases=None) -> None:
        """Point later waves at `net` (validated and packed as in __init__)."""
        w, vb, ab = _fnn_weights(net, FNN_FEAT_DIM, head_biases)
        self._weights = w
        self._net = HgFnnNet(*[t.data_ptr() for t in w], vb, ab, FNN_FEAT_DIM)

    def run(self, root_states, game_active, root_nodes, root_slots, num_candidates: int, max_root_children: int,
            c_puct: float, W: int, deterministic_non_root: bool = False, non_root_sigma: float = 4.0,
            q_penalty: float = 0.0, stats: torch.Tensor | None = None):
        """One wave of W simulations per root candidate; returns (leaf_idx,
        leaf_states, num_legal, vl_lens) of its T = W * C * B simulations.
        `stats`: hg_mcts_wave_stats' int64[4] counters to accumulate into."""
        B, C, W = self.B, int(num_candidates), int(W)
        T = W * C * B
        if T > self.capacity:
            raise ValueError(f"WavePlan: {T} simulations, capacity {self.capacity}")
        _state_rows(root_states, B)
        _dev(game_active, "game_active", torch.int8, (), B)
        _dev(root_nodes, "root_nodes", torch.int32, (), B)
        _dev(root_slots, "root_slots", torch.int32, (C,), B)
        if stats is not None:
            _dev(stats, "stats", torch.int64, (), 4)
        self._bufs.stats = stats.data_ptr() if stats is not None else None
        _check(self._lib.hg_mcts_wave_root_slots(
            ctypes.byref(self._tree), root_states.data_ptr(), game_active.data_ptr(), root_nodes.data_ptr(),
            root_slots.data_ptr(), C, int(max_root_children), float(c_puct), B, W,
            1 if deterministic_non_root else 0, float(non_root_sigma), float(q_penalty), ctypes.byref(self._net),
            ctypes.byref(self._bufs), _stream()), "mcts_wave_root_slots")
        return self.leaf_idx[:T], self.leaf_states[:T], self.num_legal[:T], self.vl_lens[:T]


def random_positions(batch_size: int, expansion_mask: int, max_ply: int, seed: int, lockstep: bool = False,
                     per_ply: bool | None = None):
    """Seeded random-play positions on the GPU (the benchmark configurations'
    generator): position i plays Philox-chosen legal moves from the empty
    board for a Philox-drawn number of plies in [0, max_ply] (or exactly
    max_ply in lockstep mode), stopping early at a result.  per_ply False:
    one launch for all plies (hg_random_play, each workgroup keeping its two
    games to their last ply); True: one legal-list launch and one move launch
    per ply (hg_random_play_step); the same result.  None: the single launch
    in lockstep mode, where every game runs to the same ply, the per-ply
    launches otherwise (games stopping at scattered plies keep the whole
    device busy that way).
    Returns (states [B,3424] u8, plies_done [B] i32)."""
    ext = load_extension()
    B = int(batch_size)
    states = ext.create_initial_states(B, expansion_mask)
    plies = torch.zeros((B,), dtype=torch.int32, device="cuda")
    lib = ext._lib
    if per_ply is None:
        per_ply = not lockstep
    if not per_ply:
        moves = torch.empty((B, MAX_LEGAL_MOVES, SIZEOF_GPU_MOVE), dtype=torch.uint8, device="cuda")
        _check(lib.hg_random_play(states.data_ptr(), moves.data_ptr(), B, int(max_ply), 1 if lockstep else 0,
                                  int(seed) & 0xFFFFFFFF, plies.data_ptr(), _stream()), "random_play")
        return states, plies
    for ply in range(int(max_ply)):
        moves, n = ext.generate_legal_moves_batch(states, B)
        _check(lib.hg_random_play_step(states.data_ptr(), moves.data_ptr(), n.data_ptr(), B, ply, int(max_ply),
                                       1 if lockstep else 0, int(seed) & 0xFFFFFFFF, plies.data_ptr(), _stream()),
               "random_play_step")
    return states, plies


def _mcts_methods():
    """MCTS entry points, bound onto HiveGpuExtension below (reference
    signatures: bindings.cpp:378-436)."""

    def mcts_select_with_root_mask_batch(self, vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt, child_init_q,
                                         game_active, root_nodes, alive_mask, max_root_children, c_puct, B, W,
                                         max_nodes, deterministic_non_root=False, non_root_sigma=4.0, q_penalty=0.0):
        B, W, M = int(B), int(W), int(max_nodes)
        tree = _tree_struct((vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt), child_init_q, B, M)
        _dev(game_active, "game_active", torch.int8, (), B)
        _dev(root_nodes, "root_nodes", torch.int32, (), B)
        _dev(alive_mask, "alive_mask", torch.int8, (int(max_root_children),), B)
        T = W * B
        out = _select_outputs(T, whole_rows=True)
        _check(self._lib.hg_mcts_select_root_mask(
            ctypes.byref(tree), game_active.data_ptr(), root_nodes.data_ptr(), alive_mask.data_ptr(),
            int(max_root_children), float(c_puct), B, W, 1 if deterministic_non_root else 0, float(non_root_sigma),
            float(q_penalty), *[o.data_ptr() for o in out], _stream()), "mcts_select_with_root_mask_batch")
        return out

    def mcts_select_with_root_slots_batch(self, vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt, child_init_q,
                                          game_active, root_nodes, root_slots, num_candidates, max_root_children,
                                          c_puct, B, W, max_nodes, deterministic_non_root=False, non_root_sigma=4.0,
                                          q_penalty=0.0):
        B, W, C, M = int(B), int(W), int(num_candidates), int(max_nodes)
        tree = _tree_struct((vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt), child_init_q, B, M)
        _dev(game_active, "game_active", torch.int8, (), B)
        _dev(root_nodes, "root_nodes", torch.int32, (), B)
        _dev(root_slots, "root_slots", torch.int32, (C,), B)
        T = W * C * B
        out = _select_outputs(T, whole_rows=True)
        _check(self._lib.hg_mcts_select_root_slots(
            ctypes.byref(tree), game_active.data_ptr(), root_nodes.data_ptr(), root_slots.data_ptr(), C,
            int(max_root_children), float(c_puct), B, W, 1 if deterministic_non_root else 0, float(non_root_sigma),
            float(q_penalty), *[o.data_ptr() for o in out], _stream()), "mcts_select_with_root_slots_batch")
        return out

    def mcts_replay_batch(self, root_states, leaf_states, move_paths, path_lengths, leaf_indices, B, total):
        B, total = int(B), int(total)
        _state_rows(root_states, B)
        _state_rows(leaf_states, total)
        _dev(move_paths, "move_paths", torch.uint8, (MAX_TREE_DEPTH, SIZEOF_GPU_MOVE), total)
        _dev(path_lengths, "path_lengths", torch.int32, (), total)
        _dev(leaf_indices, "leaf_indices", torch.int32, (), total)
        _check(self._lib.hg_mcts_replay(root_states.data_ptr(), B, leaf_states.data_ptr(), move_paths.data_ptr(),
                                        path_lengths.data_ptr(), leaf_indices.data_ptr(), total, _stream()),
               "mcts_replay_batch")

    def mcts_replay_fill_batch(self, root_states, leaf_states, move_paths, path_lengths, leaf_indices, B, total):
        """mcts_replay_batch into an uninitialised buffer: rows of idle
        simulations (leaf index < 0) are written as zero rows, as the fused
        prefix's zero-filled leaf states (game_logic.cu:1183-1254)."""
        B, total = int(B), int(total)
        _state_rows(root_states, B)
        _state_rows(leaf_states, total)
        _dev(move_paths, "move_paths", torch.uint8, (MAX_TREE_DEPTH, SIZEOF_GPU_MOVE), total)
        _dev(path_lengths, "path_lengths", torch.int32, (), total)
        _dev(leaf_indices, "leaf_indices", torch.int32, (), total)
        _check(self._lib.hg_mcts_replay_fill(root_states.data_ptr(), B, leaf_states.data_ptr(), move_paths.data_ptr(),
                                             path_lengths.data_ptr(), leaf_indices.data_ptr(), total, _stream()),
               "mcts_replay_fill_batch")

    def mcts_select_replay_legal_fnn_root_slots_batch(self, vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt,
                                                      child_init_q, root_states, game_active, root_nodes, root_slots,
                                                      num_candidates, max_root_children, c_puct, B, W, max_nodes,
                                                      deterministic_non_root=False, non_root_sigma=4.0,
                                                      q_penalty=0.0):
        """game_logic.cu:1183-1254: select -> replay -> results -> legal + features, 8-tuple."""
        leaf_idx, paths, plen, vl, vlen = self.mcts_select_with_root_slots_batch(
            vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt, child_init_q, game_active, root_nodes, root_slots,
            num_candidates, max_root_children, c_puct, B, W, max_nodes, deterministic_non_root, non_root_sigma,
            q_penalty)
        T = leaf_idx.shape[0]
        # replayed in full: rows of idle simulations are written as zero rows
        leaf_states = torch.empty((T, root_states.shape[1]), dtype=torch.uint8, device="cuda")
        self.mcts_replay_fill_batch(root_states, leaf_states, paths, plen, leaf_idx, B, T)
        results = self.check_results_batch(leaf_states, T)
        moves, n, feat = self.generate_legal_moves_and_fnn_features_batch(leaf_states, T)
        return leaf_idx, leaf_states, moves, n, feat, results, vl, vlen

    def _leaf_args(total, child_q_values, leaf_indices, leaf_states, legal_moves, num_legal, priors_per_legal,
                   results):
        _dev(child_q_values, "child_q_values", torch.float32, (MAX_LEGAL_MOVES,), total)
        _dev(leaf_indices, "leaf_indices", torch.int32, (), total)
        _state_rows(leaf_states, total)
        _dev(legal_moves, "legal_moves", torch.uint8, (MAX_LEGAL_MOVES, SIZEOF_GPU_MOVE), total)
        _dev(num_legal, "num_legal", torch.int32, (), total)
        _dev(priors_per_legal, "priors_per_legal", torch.float32, (MAX_LEGAL_MOVES,), total)
        _dev(results, "results", torch.int32, (), total)
        return [child_q_values.data_ptr(), leaf_indices.data_ptr(), leaf_states.data_ptr(), legal_moves.data_ptr(),
                num_legal.data_ptr(), priors_per_legal.data_ptr(), results.data_ptr()]

    def mcts_expand_dense_priors_batch(self, vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt, child_init_q,
                                       child_q_values, leaf_indices, leaf_states, legal_moves, num_legal,
                                       priors_per_legal, results, B, total, max_nodes):
        B, total, M = int(B), int(total), int(max_nodes)
        tree = _tree_struct((vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt), child_init_q, B, M)
        args = _leaf_args(total, child_q_values, leaf_indices, leaf_states, legal_moves, num_legal,
                          priors_per_legal, results)
        was = torch.zeros((total,), dtype=torch.int8, device="cuda")
        _check(self._lib.hg_mcts_expand_dense(ctypes.byref(tree), *args, B, total, was.data_ptr(), _stream()),
               "mcts_expand_dense_priors_batch")
        return was

    def mcts_expand_and_backprop_dense_priors_batch(self, vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt,
                                                    child_init_q, child_q_values, leaf_indices, leaf_states,
                                                    legal_moves, num_legal, priors_per_legal, results, nn_values,
                                                    vl_paths, vl_lengths, B, total, max_nodes, q_penalty):
        B, total, M = int(B), int(total), int(max_nodes)
        tree = _tree_struct((vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt), child_init_q, B, M)
        args = _leaf_args(total, child_q_values, leaf_indices, leaf_states, legal_moves, num_legal,
                          priors_per_legal, results)
        _dev(nn_values, "nn_values", torch.float32, (), total)
        _dev(vl_paths, "vl_paths", torch.int32, (MAX_TREE_DEPTH,), total)
        _dev(vl_lengths, "vl_lengths", torch.int32, (), total)
        # the root children's simulations in parallel (hg_mcts_expand_backprop_dense_ws): same tree
        ws = torch.empty((max(1, (int(self._lib.hg_mcts_expand_backprop_dense_workspace(B, total)) + 3) // 4),),
                         dtype=torch.int32, device="cuda")
        _check(self._lib.hg_mcts_expand_backprop_dense_ws(
            ctypes.byref(tree), *args, nn_values.data_ptr(), vl_paths.data_ptr(), vl_lengths.data_ptr(),
            float(q_penalty), B, total, ws.data_ptr(), _stream()), "mcts_expand_and_backprop_dense_priors_batch")

    # ---- legacy action-space engine (bindings.cpp:378-389; twelve tree tensors, no child_init_q,
    # which these kernels never touch: any [B, M] f32 array fills its slot) ----
    def mcts_select_batch(self, vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt, game_active, root_nodes, c_puct,
                          B, W, max_nodes):
        """game_logic.cu:961-993 -> (leaf_idx, move_paths, path_lens, vl_paths, vl_lens), T = W * B."""
        B, W, M = int(B), int(W), int(max_nodes)
        tree = _tree_struct((vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt), tv, B, M)
        _dev(game_active, "game_active", torch.int8, (), B)
        _dev(root_nodes, "root_nodes", torch.int32, (), B)
        out = _select_outputs(W * B)
        _check(self._lib.hg_mcts_select(ctypes.byref(tree), game_active.data_ptr(), root_nodes.data_ptr(),
                                        float(c_puct), B, W, *[o.data_ptr() for o in out], _stream()),
               "mcts_select_batch")
        return out

    def _legacy_leaf(total, leaf_indices, leaf_states, legal_moves, num_legal, action_probs, results):
        _dev(leaf_indices, "leaf_indices", torch.int32, (), total)
        _state_rows(leaf_states, total)
        _dev(legal_moves, "legal_moves", torch.uint8, (MAX_LEGAL_MOVES, SIZEOF_GPU_MOVE), total)
        _dev(num_legal, "num_legal", torch.int32, (), total)
        _dev(action_probs, "action_probs", torch.float32, (ACTION_SPACE_SIZE,), total)
        _dev(results, "results", torch.int32, (), total)
        return [leaf_indices.data_ptr(), leaf_states.data_ptr(), legal_moves.data_ptr(), num_legal.data_ptr(),
                action_probs.data_ptr(), results.data_ptr()]

    def mcts_expand_batch(self, vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt, leaf_indices, leaf_states,
                          legal_moves, num_legal, action_probs, results, B, total, max_nodes):
        """game_logic.cu:1018-1045 -> was_expanded [total] int8."""
        B, total, M = int(B), int(total), int(max_nodes)
        tree = _tree_struct((vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt), tv, B, M)
        args = _legacy_leaf(total, leaf_indices, leaf_states, legal_moves, num_legal, action_probs, results)
        was = torch.zeros((total,), dtype=torch.int8, device="cuda")
        _check(self._lib.hg_mcts_expand(ctypes.byref(tree), *args, B, total, was.data_ptr(), _stream()),
               "mcts_expand_batch")
        return was

    def mcts_backprop_batch(self, vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt, leaf_indices, nn_values,
                            vl_paths, vl_lengths, was_expanded, B, total, max_nodes):
        """game_logic.cu:1328-1349, in place."""
        B, total, M = int(B), int(total), int(max_nodes)
        tree = _tree_struct((vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt), tv, B, M)
        _dev(leaf_indices, "leaf_indices", torch.int32, (), total)
        _dev(nn_values, "nn_values", torch.float32, (), total)
        _dev(vl_paths, "vl_paths", torch.int32, (MAX_TREE_DEPTH,), total)
        _dev(vl_lengths, "vl_lengths", torch.int32, (), total)
        _dev(was_expanded, "was_expanded", torch.int8, (), total)
        _check(self._lib.hg_mcts_backprop(ctypes.byref(tree), leaf_indices.data_ptr(), nn_values.data_ptr(),
                                          vl_paths.data_ptr(), vl_lengths.data_ptr(), was_expanded.data_ptr(), B,
                                          total, _stream()), "mcts_backprop_batch")

    def mcts_expand_and_backprop_batch(self, vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt, leaf_indices,
                                       leaf_states, legal_moves, num_legal, action_probs, results, nn_values,
                                       vl_paths, vl_lengths, B, total, max_nodes):
        """game_logic.cu:1053-1080, in place."""
        B, total, M = int(B), int(total), int(max_nodes)
        tree = _tree_struct((vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt), tv, B, M)
        args = _legacy_leaf(total, leaf_indices, leaf_states, legal_moves, num_legal, action_probs, results)
        _dev(nn_values, "nn_values", torch.float32, (), total)
        _dev(vl_paths, "vl_paths", torch.int32, (MAX_TREE_DEPTH,), total)
        _dev(vl_lengths, "vl_lengths", torch.int32, (), total)
        _check(self._lib.hg_mcts_expand_backprop(ctypes.byref(tree), *args, nn_values.data_ptr(),
                                                 vl_paths.data_ptr(), vl_lengths.data_ptr(), B, total, _stream()),
               "mcts_expand_and_backprop_batch")

    def mcts_extract_policy_batch(self, vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt, move_numbers, root_nodes,
                                  temperature, temp_drop_move, pruning_threshold, B, max_nodes):
        """game_logic.cu:1355-1379 -> policies [B, 85834] f32."""
        B, M = int(B), int(max_nodes)
        tree = _tree_struct((vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt), tv, B, M)
        _dev(move_numbers, "move_numbers", torch.int32, (), B)
        _dev(root_nodes, "root_nodes", torch.int32, (), B)
        pol = torch.empty((B, ACTION_SPACE_SIZE), dtype=torch.float32, device="cuda")
        _check(self._lib.hg_mcts_extract_policy(ctypes.byref(tree), move_numbers.data_ptr(), root_nodes.data_ptr(),
                                                float(temperature), int(temp_drop_move), float(pruning_threshold), B,
                                                pol.data_ptr(), _stream()), "mcts_extract_policy_batch")
        return pol

    def mcts_apply_root_noise(self, vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt, noise, root_nodes,
                              max_children_pad, dir_eps, root_policy_temp, B, max_nodes):
        B, M, pad = int(B), int(max_nodes), int(max_children_pad)
        # the noise kernel never touches child_init_q; any [B, M] f32 array fills the slot
        tree = _tree_struct((vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt), tv, B, M)
        _dev(noise, "noise", torch.float32, (pad,), B)
        _dev(root_nodes, "root_nodes", torch.int32, (), B)
        _check(self._lib.hg_mcts_root_noise(ctypes.byref(tree), noise.data_ptr(), root_nodes.data_ptr(), pad,
                                            float(dir_eps), float(root_policy_temp), B, _stream()),
               "mcts_apply_root_noise")

    def mcts_wave_stats(self, leaf_indices, num_legal, vl_lengths, total, stats):
        """Search counters of one wave (no counterpart in the reference):
        stats int64[4] += (leaves reached, their legal counts, their virtual-loss
        path lengths, rows), in stream order."""
        total = int(total)
        _dev(leaf_indices, "leaf_indices", torch.int32, (), total)
        _dev(num_legal, "num_legal", torch.int32, (), total)
        _dev(vl_lengths, "vl_lengths", torch.int32, (), total)
        _dev(stats, "stats", torch.int64, (), 4)
        _check(self._lib.hg_mcts_wave_stats(leaf_indices.data_ptr(), num_legal.data_ptr(), vl_lengths.data_ptr(),
                                            total, stats.data_ptr(), _stream()), "mcts_wave_stats")

    def mcts_reset_trees(self, vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt, child_init_q, reset, root_node,
                         B, max_nodes):
        """Hard rebase (_reroot_tree, fnn_mcts_orchestrator.py:1122-1142) of
        the games with reset[g] (bool or int8 [B]); extension entry point."""
        B, M = int(B), int(max_nodes)
        tree = _tree_struct((vc, tv, pr, pa, vq, mb, ai, fc, nc, it, tv2, cnt), child_init_q, B, M)
        if reset.dtype == torch.bool:
            reset = reset.view(torch.int8)
        _dev(reset, "reset", torch.int8, (), B)
        _dev(root_node, "root_node", torch.int32, (), B)
        _check(self._lib.hg_mcts_reset_trees(ctypes.byref(tree), reset.data_ptr(), root_node.data_ptr(), B,
                                             _stream()), "mcts_reset_trees")

    return {k: v for k, v in locals().items() if k.startswith("mcts_")}


for _name, _fn in _mcts_methods().items():
    setattr(HiveGpuExtension, _name, _fn)


_extension = None


# Entry points of the reference module outside this engine's path (bindings.cpp:254-476):
# GNN / transformer token encoders, mobility labels, the PRS classifier, the
# endgame hit mask, the experimental fused self-play kernel and the
# move-generation profiling hooks.  They are present so a caller gets a clear
# error instead of an AttributeError.
_OUT_OF_SCOPE = (
    "compute_mobility_batch", "debug_tactical_state_batch", "encode_states_batch", "endgame_hit_mask_batch",
    "fnn_selfplay_batch", "generate_legal_moves_and_hybrid_root_features_batch", "get_movegen_profile",
    "hybrid_gnn_encode_batch", "hybrid_gnn_encode_with_moves_batch", "hybrid_transformer_encode_with_moves_batch",
    "hybrid_transformer_move_features_batch", "prs_v2_classify_batch", "reset_movegen_profile",
)


def _out_of_scope(name):
    def fn(self, *args, **kwargs):
        raise NotImplementedError(
            f"{name} is not provided by the MI355X engine: it serves the GNN/transformer, PRS, mobility-label "
            "or profiling lines of the reference, outside the move-generation / FNN / MCTS path built here")
    fn.__name__ = name
    return fn


for _name in _OUT_OF_SCOPE:
    setattr(HiveGpuExtension, _name, _out_of_scope(_name))


def load_extension() -> HiveGpuExtension:
    """Idempotent: load libhive_gpu.so, initialise tables, return the extension."""
    global _extension
    if _extension is None:
        if not torch.cuda.is_available():
            raise RuntimeError("hive_gpu needs a HIP device (torch.cuda.is_available() is False)")
        ext = HiveGpuExtension(load_library())
        ext.initialize_tables()
        _extension = ext
    return _extension
