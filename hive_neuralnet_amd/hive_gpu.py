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
    "hg_extract_fnn_features": [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_void_p, _c_void_p],
    "hg_legal_moves_to_actions": [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_void_p, _c_void_p],
    "hg_compute_centroids": [_c_void_p, _c_i64, _c_void_p, _c_void_p],
    "hg_fnn_successor_features": [_c_void_p, _c_void_p, _c_i64, _c_void_p, _c_void_p, _c_i64, _c_void_p,
                                  _c_void_p],
    "hg_queen_escape_flags": [_c_void_p, _c_i64, _c_void_p, _c_void_p],
    "hg_random_play_step": [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_int, _c_int, _c_int, ctypes.c_uint32,
                            _c_void_p, _c_void_p],
}

_lib = None
_lib_lock = threading.Lock()


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
        _lib = lib
        return lib


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _check(err: int, what: str) -> None:
    if err != 0:
        raise RuntimeError(f"{what}: HIP error {err}")


def _dev(t: torch.Tensor, name: str, dtype: torch.dtype, inner: tuple, rows: int) -> torch.Tensor:
    """Validate a device tensor: dtype, trailing shape, >= rows rows, contiguous."""
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if inner and tuple(t.shape[-len(inner):]) != tuple(inner):
        if t.numel() != 0 and t.numel() % max(1, int(torch.tensor(inner).prod())) == 0:
            t = t.reshape(-1, *inner)
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

    def generate_legal_moves_features_actions_batch(self, states: torch.Tensor, batch_size: int):
        """Fused: (moves, num_legal, features, action_indices) in one pass."""
        B = int(batch_size)
        states = _state_rows(states, B)
        moves = torch.empty((B, MAX_LEGAL_MOVES, SIZEOF_GPU_MOVE), dtype=torch.uint8, device="cuda")
        n = torch.empty((B,), dtype=torch.int32, device="cuda")
        feat = torch.empty((B, FNN_FEAT_DIM), dtype=torch.float32, device="cuda")
        act = torch.empty((B, MAX_LEGAL_MOVES), dtype=torch.int32, device="cuda")
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
                                     num_actions: int) -> torch.Tensor:
        N = int(num_actions)
        states = _dev(states, "states", torch.uint8, (SIZEOF_HIVE_STATE,), 0)
        legal_moves = _dev(legal_moves, "legal_moves", torch.uint8, (MAX_LEGAL_MOVES, SIZEOF_GPU_MOVE), 0)
        action_to_root = _dev(action_to_root, "action_to_root", torch.int64, (), N)
        move_indices = _dev(move_indices, "move_indices", torch.int64, (), N)
        feat = torch.empty((N, FNN_FEAT_DIM), dtype=torch.float32, device="cuda")
        roots = min(states.numel() // SIZEOF_HIVE_STATE, legal_moves.numel() // (MAX_LEGAL_MOVES * SIZEOF_GPU_MOVE))
        _check(self._lib.hg_fnn_successor_features(states.data_ptr(), legal_moves.data_ptr(), roots,
                                                   action_to_root.data_ptr(), move_indices.data_ptr(), N,
                                                   feat.data_ptr(), _stream()), "fnn_successor_features_batch")
        return feat

    def queen_escape_flags_batch(self, states: torch.Tensor, batch_size: int) -> torch.Tensor:
        B = int(batch_size)
        states = _state_rows(states, B)
        out = torch.empty((B,), dtype=torch.uint8, device="cuda")
        _check(self._lib.hg_queen_escape_flags(states.data_ptr(), B, out.data_ptr(), _stream()),
               "queen_escape_flags_batch")
        return out


def random_positions(batch_size: int, expansion_mask: int, max_ply: int, seed: int, lockstep: bool = False):
    """Seeded random-play positions on the GPU (the benchmark configurations'
    generator): position i plays Philox-chosen legal moves from the empty
    board for a Philox-drawn number of plies in [0, max_ply] (or exactly
    max_ply in lockstep mode), stopping early at a result.
    Returns (states [B,3424] u8, plies_done [B] i32)."""
    ext = load_extension()
    B = int(batch_size)
    states = ext.create_initial_states(B, expansion_mask)
    plies = torch.zeros((B,), dtype=torch.int32, device="cuda")
    lib = ext._lib
    for ply in range(int(max_ply)):
        moves, n = ext.generate_legal_moves_batch(states, B)
        _check(lib.hg_random_play_step(states.data_ptr(), moves.data_ptr(), n.data_ptr(), B, ply, int(max_ply),
                                       1 if lockstep else 0, int(seed) & 0xFFFFFFFF, plies.data_ptr(), _stream()),
               "random_play_step")
    return states, plies


_extension = None


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
