"""Write the golden vectors under tests/golden/ from the reference's own engine.

Run in the container that mounts the reference (``make -C oracle ref`` first):

    python tests/golden/make_golden.py

Inputs are seeded Philox random-play positions.  Every output array comes
from the reference's own C++ (hive_gpu/csrc/cpu_native.cpp compiled by
oracle/ref_capi.cpp); the positions themselves are re-derived by replaying
the Philox choices through the reference's legal-move lists, so the
generator is pinned too.  The fixtures are data only (inputs and expected
outputs); no reference source is stored.
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import MAX_LEGAL, Oracle, Reference  # noqa: E402

SEED = 0x5EED
OUT = os.path.dirname(os.path.abspath(__file__))

# (name, count, expansion mask, max ply): small stand-ins of configs C1, C2, C3
SETS = [("c1", 256, 0, 60), ("c2", 256, 0, 120), ("c3", 384, 7, 150)]


def replay_positions(ref: Reference, orc: Oracle, count: int, mask: int, max_ply: int, seed: int):
    """Random play with the reference's own lists and apply (pins the generator)."""
    states = np.zeros((count, 3424), np.uint8)
    plies = np.zeros(count, np.int32)
    for i in range(count):
        s = ref.init_state(mask)
        target = int(orc.philox(seed, 0, [i, 0, 0, 0])[0]) % (max_ply + 1)
        done = 0
        for p in range(target):
            if s[3415] != 0:
                break
            moves, n = ref.legal_moves(s)
            u = int(orc.philox(seed, 0, [i, p + 1, 0, 0])[0])
            pick = (u * n) >> 32
            s = ref.apply_move(s, moves[pick])
            done += 1
        states[i] = s
        plies[i] = done
    return states, plies


def main() -> None:
    ref = Reference.load()
    if ref is None:
        raise SystemExit("oracle/_ref/libhive_ref.so missing: run `make -C oracle ref`")
    orc = Oracle()
    for name, count, mask, max_ply in SETS:
        states, plies = replay_positions(ref, orc, count, mask, max_ply, SEED)
        moves, n, feat = ref.batch_legal_features(states, threads=1)
        compact = np.zeros((count, MAX_LEGAL, 6), np.uint8)
        ncompact = np.zeros(count, np.int32)
        ap = np.zeros((count, 9), np.uint64)
        qesc = np.zeros(count, np.uint8)
        for i in range(count):
            compact[i], ncompact[i] = ref.fnn_feature_moves(states[i])
            ap[i] = ref.articulation(states[i])
            qesc[i] = ref.queen_escape(states[i])
        # successors of the first 48 positions: every legal move
        R = min(48, count)
        roots = np.repeat(np.arange(R), n[:R]).astype(np.int64)
        idx = np.concatenate([np.arange(k) for k in n[:R]]).astype(np.int64)
        succ = ref.batch_successor_features(states, moves, roots, idx, full_list=False, threads=1)
        succ_full = ref.batch_successor_features(states, moves, roots, idx, full_list=True, threads=1)
        # successor states (apply_move only) for a hash-level pin of apply
        child = np.stack([ref.apply_move(states[r], moves[r, k]) for r, k in zip(roots[:512], idx[:512])])
        np.savez_compressed(
            os.path.join(OUT, f"golden_{name}.npz"),
            seed=np.uint32(SEED), mask=np.int32(mask), max_ply=np.int32(max_ply),
            states=states, plies=plies, moves=moves, n=n, features=feat,
            compact=compact, ncompact=ncompact, ap=ap, queen_escape=qesc,
            succ_root=roots, succ_idx=idx, succ_features=succ, succ_features_full=succ_full,
            child_states=child,
        )
        print(name, "positions", count, "mean legal", float(n.mean()), "successors", len(roots))
    # lockstep self-play (config C4 shape, small): final states by reference replay
    G, P = 24, 300
    finals = np.zeros((G, 3424), np.uint8)
    plies = np.zeros(G, np.int32)
    for g in range(G):
        s = ref.init_state(0)
        done = 0
        for p in range(P):
            if s[3415] != 0:
                break
            moves, n = ref.legal_moves(s)
            u = int(orc.philox(SEED, 0, [g, p + 1, 0, 0])[0])
            s = ref.apply_move(s, moves[(u * n) >> 32])
            done += 1
        finals[g] = s
        plies[g] = done
    np.savez_compressed(os.path.join(OUT, "golden_c4.npz"), seed=np.uint32(SEED), max_ply=np.int32(P),
                        finals=finals, plies=plies)
    print("c4 games", G, "results", np.bincount(finals[:, 3415], minlength=4).tolist())


if __name__ == "__main__":
    main()
