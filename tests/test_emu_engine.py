"""The engine's device programs run on the CPU under the wave emulator.

tests/emu/ compiles hive_neuralnet_amd/csrc/hive_phases.hpp for the host,
running each 64-lane wave as 64 threads with barrier-based shuffles and
ballots.  This checks the device logic (order of emission, features,
compact successor summaries, queen escape) against the reference's golden
vectors without a GPU; the GPU tests check the compiled HIP library itself.
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT, load_golden

EMU = os.path.join(ROOT, "tests", "emu")


@pytest.fixture(scope="module")
def emu():
    subprocess.run(["make", "-s", "-C", EMU], check=True)
    return ctypes.CDLL(os.path.join(EMU, "libwave_emu.so"))


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


@pytest.mark.parametrize("name", ["c1", "c2", "c3"])
def test_emulated_legal_features(emu, oracle, name):
    g = load_golden(name)
    st = np.ascontiguousarray(g["states"][:47])
    B = len(st)
    mv = np.zeros((B, 256, 6), np.uint8)
    n = np.zeros(B, np.int32)
    f = np.zeros((B, 122), np.float32)
    a = np.zeros((B, 256), np.int32)
    emu.emu_legal(_p(st), ctypes.c_int64(B), _p(mv), _p(n), _p(f), _p(a))
    assert np.array_equal(n, g["n"][:B])
    assert np.array_equal(mv, g["moves"][:B])
    assert np.array_equal(f.view(np.uint32), g["features"][:B].view(np.uint32))
    _, _, _, oa = oracle.batch_legal_features_actions(st)
    assert np.array_equal(a, oa)


@pytest.mark.parametrize("name", ["c2", "c3"])
def test_emulated_successors_queen_escape(emu, name):
    g = load_golden(name)
    k = 160
    roots = np.ascontiguousarray(g["succ_root"][:k])
    idx = np.ascontiguousarray(g["succ_idx"][:k])
    st = np.ascontiguousarray(g["states"])
    mv = np.ascontiguousarray(g["moves"])
    f = np.zeros((k, 122), np.float32)
    emu.emu_successor(_p(st), _p(mv), _p(roots), _p(idx), ctypes.c_int64(k), _p(f))
    assert np.array_equal(f.view(np.uint32), g["succ_features"][:k].view(np.uint32))
    q = np.zeros(64, np.uint8)
    emu.emu_queen_escape(_p(st), ctypes.c_int64(64), _p(q))
    assert np.array_equal(q, g["queen_escape"][:64])


def test_emulated_root_tactical_probe(emu):
    """hive_probe.hpp's group programs, orchestrated as hive_probe.hip's
    launches, against the reference's probe vectors: four positions of every
    outcome kind with all stages enabled (the emulator runs a move generation
    in ~10 ms, so the full fixture is left to the GPU test)."""
    g = load_golden("probe")
    kinds = g["kinds"]
    sel = np.concatenate([np.nonzero(kinds == k)[0][:4] for k in sorted(set(kinds.tolist()))])
    st, lm, nl, pr = (np.ascontiguousarray(g[k][sel]) for k in ("states", "legal", "nlegal", "priors"))
    B = len(st)
    j = 0
    assert tuple(g["flags"][j]) == (1, 1, 1)
    win = np.zeros(B, np.int64)
    allowed = np.zeros((B, 256), np.uint8)
    forced = np.zeros(B, np.uint8)
    emu.emu_root_probe(_p(st), _p(lm), _p(nl), _p(pr), ctypes.c_int64(B), 1, 1, 1, _p(win), _p(allowed),
                       _p(forced))
    assert np.array_equal(win, g["win"][j][sel]), np.nonzero(win != g["win"][j][sel])[0][:8]
    assert np.array_equal(forced, g["forced"][j][sel])
    assert np.array_equal(allowed, g["allowed"][j][sel])
