"""CPU-side checks of the drop-in boundary (no compute calls, no GPU needed)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hive_gpu.h")
LIB = os.path.join(ROOT, "hive_neuralnet_amd", "libhive_gpu.so")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^(?:int|int64_t) (hg_\w+)\(", text, flags=re.M)))


def test_header_declares_entry_points():
    names = _declared()
    assert "hg_generate_legal_moves" in names and "hg_fnn_successor_features" in names
    assert len(names) >= 14


@pytest.mark.skipif(not os.path.exists(LIB), reason="libhive_gpu.so not built (run python -m hive_neuralnet_amd.build)")
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(LIB)
    for name in _declared():
        assert hasattr(lib, name), name
    lib.hg_abi_version.restype = ctypes.c_int
    assert lib.hg_abi_version() == 1  # pure host call, no device work


def test_python_binding_matches_header():
    from hive_neuralnet_amd import hive_gpu
    assert sorted(list(hive_gpu._SIGS) + list(hive_gpu._SIGS_I64)) == _declared()


def test_reference_surface_names():
    """Every entry point the reference's hive_fnn callers use exists (bindings.cpp:254-476)."""
    from hive_neuralnet_amd.hive_gpu import HiveGpuExtension
    for name in ["initialize_tables", "create_initial_states", "generate_legal_moves_batch",
                 "apply_moves_batch", "check_results_batch", "extract_fnn_features_batch",
                 "generate_legal_moves_and_fnn_features_batch", "fnn_successor_features_batch",
                 "legal_moves_to_actions_batch", "compute_centroids_batch", "queen_escape_flags_batch",
                 "root_tactical_probe_batch", "generate_legal_mask_batch", "generate_legal_moves_and_mask_batch",
                 "mcts_select_batch", "mcts_replay_batch", "mcts_expand_batch", "mcts_backprop_batch",
                 "mcts_expand_and_backprop_batch", "mcts_extract_policy_batch", "mcts_apply_root_noise",
                 "mcts_select_with_root_mask_batch", "mcts_select_with_root_slots_batch",
                 "mcts_select_replay_legal_fnn_root_slots_batch", "mcts_expand_dense_priors_batch",
                 "mcts_expand_and_backprop_dense_priors_batch"]:
        assert callable(getattr(HiveGpuExtension, name)), name


def test_no_fallback_without_device(monkeypatch):
    import torch
    from hive_neuralnet_amd import hive_gpu
    if torch.cuda.is_available():
        pytest.skip("device present")
    monkeypatch.setattr(hive_gpu, "_extension", None)
    with pytest.raises(RuntimeError):
        hive_gpu.load_extension()


def test_reference_surface_complete():
    """Every entry point of the reference module (bindings.cpp) exists on the
    extension object; those outside this engine's path raise
    NotImplementedError with a message."""
    import pytest
    from hive_neuralnet_amd import hive_gpu
    names = ["initialize_tables", "create_initial_states", "apply_moves_batch", "check_results_batch",
             "generate_legal_moves_batch", "generate_legal_moves_and_fnn_features_batch",
             "fnn_successor_features_batch", "legal_moves_to_actions_batch", "compute_centroids_batch",
             "mcts_select_with_root_slots_batch", "mcts_expand_and_backprop_dense_priors_batch",
             "root_tactical_probe_batch", "queen_escape_flags_batch"] + list(hive_gpu._OUT_OF_SCOPE)
    for n in names:
        assert callable(getattr(hive_gpu.HiveGpuExtension, n, None)), n
    ext = hive_gpu.HiveGpuExtension.__new__(hive_gpu.HiveGpuExtension)
    with pytest.raises(NotImplementedError, match="not provided"):
        ext.encode_states_batch(None, 1)
