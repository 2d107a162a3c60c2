"""The oracle against the reference's own CPU build at the configs' full sizes.

oracle/_ref/libhive_ref.so is the reference's hive_gpu/csrc/cpu_native.cpp
compiled here (oracle/Makefile target `ref`); it exists only in the build
container, so these tests skip elsewhere.  Positions come from the oracle's
seeded Philox generator (the generator itself is pinned by the golden
vectors: its positions are re-derived through the reference's lists).

* C1 (1,024, mask 0, plies U[0,60]), C2 (65,536, mask 0, U[0,120]) and C3
  (65,536, mask 7, U[0,150]): legal lists (order and bytes), counts and the
  122 features bit for bit;
* successor features (compact and full lists) of every legal move of 4,096
  roots of C2 and of C3;
* queen-escape flags of the children of 4,096 C3 roots.
"""
import numpy as np
import pytest

from oracle import Reference

REF = Reference.load()
pytestmark = pytest.mark.skipif(REF is None, reason="oracle/_ref not built (needs /root/reference): "
                                                     "make -C oracle ref")

SEED = 0x5EED
CONFIGS = {"c1": (1024, 0, 60), "c2": (65536, 0, 120), "c3": (65536, 7, 150)}


@pytest.fixture(scope="module")
def positions(oracle):
    return {k: oracle.generate_positions(B, mask, ply, SEED)[0] for k, (B, mask, ply) in CONFIGS.items()}


def _bits(x):
    return np.ascontiguousarray(x).view(np.uint32)


@pytest.mark.parametrize("name", ["c1", "c2", "c3"])
def test_full_size_lists_and_features(oracle, positions, name):
    st = positions[name]
    om, on, of, _ = oracle.batch_legal_features_actions(st, want_actions=False)
    rm, rn, rf = REF.batch_legal_features(st)
    assert np.array_equal(on, rn)
    assert np.array_equal(om, rm)
    assert np.array_equal(_bits(of), _bits(rf))


@pytest.mark.parametrize("name", ["c2", "c3"])
@pytest.mark.parametrize("full", [False, True], ids=["compact", "full"])
def test_successor_features(oracle, positions, name, full):
    st = positions[name][:4096]
    legal, n, _, _ = oracle.batch_legal_features_actions(st, want_features=False, want_actions=False)
    a2r = np.repeat(np.arange(st.shape[0]), n).astype(np.int64)
    mi = np.concatenate([np.arange(k) for k in n]).astype(np.int64)
    assert a2r.shape[0] > 100_000
    want = REF.batch_successor_features(st, legal, a2r, mi, full_list=full)
    got = oracle.batch_successor_features(st, legal, a2r, mi, full_list=full)
    assert np.array_equal(_bits(got), _bits(want))


def test_queen_escape_children(oracle, positions):
    st = positions["c3"][:4096]
    legal, n, _, _ = oracle.batch_legal_features_actions(st, want_features=False, want_actions=False)
    kids = np.stack([oracle.apply_move(st[r], legal[r, i]) for r in range(0, 4096, 7) for i in range(int(n[r]))])
    assert kids.shape[0] > 5000
    want = np.array([REF.queen_escape(k) for k in kids])
    assert np.array_equal(oracle.batch_queen_escape(kids), want.astype(oracle.batch_queen_escape(kids[:1]).dtype))
