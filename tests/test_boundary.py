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


def test_struct_layouts_match_header(tmp_path):
    """The ctypes mirrors of the header's structs (hg_tree, hg_fnn_net,
    hg_wave_buffers) have the C compiler's field offsets and sizes: the
    header compiled by gcc prints offsetof / sizeof of every field."""
    import shutil
    import subprocess
    from hive_neuralnet_amd import hive_gpu
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    mirrors = {"hg_tree": hive_gpu.HgTree, "hg_fnn_net": hive_gpu.HgFnnNet, "hg_wave_buffers": hive_gpu.HgWaveBuffers}
    lines = []
    for cname, cls in mirrors.items():
        lines.append(f'printf("{cname} %zu\\n", sizeof({cname}));')
        for f, _ in cls._fields_:
            lines.append(f'printf("{cname}.{f} %zu\\n", offsetof({cname}, {f}));')
    src = tmp_path / "layout.c"
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "hive_gpu.h"\nint main(void) {\n'
                   + "\n".join(lines) + "\nreturn 0;\n}\n")
    exe = tmp_path / "layout"
    subprocess.run([gcc, "-std=c99", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = dict(line.split() for line in subprocess.run([str(exe)], check=True, capture_output=True,
                                                         text=True).stdout.splitlines())
    for cname, cls in mirrors.items():
        assert int(got[cname]) == ctypes.sizeof(cls), cname
        for f, _ in cls._fields_:
            assert int(got[f"{cname}.{f}"]) == getattr(cls, f).offset, f"{cname}.{f}"


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


@pytest.mark.skipif(not os.path.exists(LIB), reason="libhive_gpu.so not built (run python -m hive_neuralnet_amd.build)")
def test_probe_rejects_misaligned_workspace():
    """hg_root_tactical_probe keeps a 64-bit atomic counter in its workspace:
    a workspace that is not 8-byte aligned, or missing, is refused with
    hipErrorInvalidValue (1) on the host, before any launch (so this runs
    without a GPU: no device memory is touched)."""
    lib = ctypes.CDLL(LIB)
    f = lib.hg_root_tactical_probe
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int64] + [ctypes.c_int] * 3 + [ctypes.c_void_p] * 5
    buf = (ctypes.c_int32 * 64)()
    base = ctypes.addressof(buf)
    aligned = (base + 7) & ~7
    for ws in (aligned + 4, aligned + 2, 0):
        assert f(aligned, aligned, aligned, aligned, 1, 1, 1, 1, aligned, aligned, aligned, ws or None, None) == 1
