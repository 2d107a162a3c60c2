"""Write tests/golden/golden_probe.npz: root tactical probe vectors from the
reference's own engine.

Run in the container that mounts the reference (``make -C oracle ref`` first):

    python tests/golden/make_golden_probe.py

Inputs: seeded random-play positions (this repository's Philox generator, the
same one the other fixtures pin) sampled by what the probe does with them --
no tactic, an immediate win, a two-move forced win, a screened move list, a
forced random move -- plus positions where no gate applies.  The legal lists,
the immediate-win flags and every probe output come from the reference
(oracle/ref_capi.cpp over hive_gpu/csrc, composed as
root_tactical_probe_kernel, game_logic.cu:290-397).  Priors are multiples of
1/8 so that ties between winning moves occur.  Data only.
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import MAX_LEGAL, Oracle, Reference  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden_probe.npz")
FLAGS = [(1, 1, 1), (1, 0, 1), (0, 1, 0), (0, 0, 1)]
PER_KIND = {"none": 60, "screened": 70, "w1": 60, "w2": 70, "forced": 24, "ungated": 30}


def main() -> None:
    ref = Reference.load()
    if ref is None:
        raise SystemExit("oracle/_ref/libhive_ref.so missing: run `make -C oracle ref`")
    orc = Oracle()
    rng = np.random.default_rng(0x7AC)
    picked = {k: [] for k in PER_KIND}
    for mask, max_ply, seed in [(0, 150, 11), (7, 150, 12), (0, 300, 13), (7, 300, 14), (0, 220, 15), (7, 220, 16)]:
        st, _ = orc.generate_positions(60000, mask, max_ply, seed)
        turn = st[:, 3412].astype(np.int64) | (st[:, 3413].astype(np.int64) << 8)
        me = turn & 1
        for i in rng.permutation(len(st)):
            s = st[i]
            if s[3415] != 0:
                continue
            opp, own = orc.surround_count(s, 1 - me[i]), orc.surround_count(s, me[i])
            mv, n = ref.legal_moves(s)
            pr = (rng.integers(0, 8, size=MAX_LEGAL) / 8.0).astype(np.float32)
            if not (opp >= 4 or own == 5):
                kind = "ungated"
            else:
                w, a, f = ref.root_tactical_probe(s, mv, n, pr)
                if f:
                    kind = "forced"
                elif w >= 0:
                    kind = "w1" if ref.apply_move(s, mv[w])[3415] != 0 else "w2"
                elif n > 0 and a[:n].min() == 0:
                    kind = "screened"
                else:
                    kind = "none"
            if len(picked[kind]) < PER_KIND[kind]:
                picked[kind].append((s.copy(), mv, n, pr))
            if all(len(picked[k]) >= PER_KIND[k] for k in PER_KIND):
                break
    rows = [r for k in PER_KIND for r in picked[k]]
    kinds = np.array([k for k in PER_KIND for _ in picked[k]])
    states = np.stack([r[0] for r in rows])
    legal = np.stack([r[1] for r in rows])
    nlegal = np.array([r[2] for r in rows], np.int32)
    priors = np.stack([r[3] for r in rows])
    B = len(rows)
    win = np.zeros((len(FLAGS), B), np.int64)
    allowed = np.zeros((len(FLAGS), B, MAX_LEGAL), np.uint8)
    forced = np.zeros((len(FLAGS), B), np.uint8)
    for j, (f1, f2, f3) in enumerate(FLAGS):
        for i in range(B):
            win[j, i], allowed[j, i], forced[j, i] = ref.root_tactical_probe(states[i], legal[i], nlegal[i],
                                                                             priors[i], f1, f2, f3)
    # has_immediate_surround_win_for_current_player on the children of the first 40 roots
    kids, iw = [], []
    for i in range(min(40, B)):
        for k in range(nlegal[i]):
            c = ref.apply_move(states[i], legal[i, k])
            kids.append(c)
            iw.append(ref.immediate_win(c))
    np.savez_compressed(OUT, states=states, legal=legal, nlegal=nlegal, priors=priors, kinds=kinds,
                        flags=np.array(FLAGS, np.int32), win=win, allowed=allowed, forced=forced,
                        child_states=np.stack(kids), child_immediate_win=np.array(iw, np.uint8))
    print({k: len(v) for k, v in picked.items()}, "children", len(kids), "->", OUT)


if __name__ == "__main__":
    main()
