"""Parity of the HIP engine (through the C-ABI) with the reference semantics.

Checks, all bit-exact (features compared as float32 bit patterns):
  * golden vectors written by the reference's own engine (tests/golden/);
  * the CPU oracle on seeded Philox positions at the configurations' full
    sizes (C2: 65,536 base positions, plies U[0,120]; C3: 65,536 positions
    with mosquito/ladybug/pillbug, plies U[0,150]);
  * the GPU position generator against the oracle's, and lockstep random
    self-play finals against reference replays (C4 shape);
  * edge cases: empty batch, finished games, caller-supplied lists.
"""
import numpy as np
import pytest
import torch

from conftest import load_golden

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ext():
    from hive_neuralnet_amd import hive_gpu
    return hive_gpu.load_extension()


def _cuda(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _bits(f):
    return np.ascontiguousarray(f).view(np.uint32)


def test_constants(ext):
    assert ext.BOARD_SIZE == 23 and ext.NUM_CELLS == 529 and ext.MAX_LEGAL_MOVES == 256
    assert ext.SIZEOF_HIVE_STATE == 3424 and ext.SIZEOF_GPU_MOVE == 6 and ext.FNN_FEAT_DIM == 122
    assert ext.ACTION_SPACE_SIZE == 85834 and ext.PASS_ACTION_INDEX == 85833 and ext.MOVEMENT_OFFSET == 2312


def test_initial_states(ext, oracle):
    for mask in range(8):
        s = ext.create_initial_states(5, mask).cpu().numpy()
        for row in s:
            assert np.array_equal(row, oracle.init_state(mask))
    # tests/test_gpu_move_gen.py:148-160 -- 4 placements at turn 0, results 0
    st = ext.create_initial_states(8)
    moves, n = ext.generate_legal_moves_batch(st, 8)
    assert n.cpu().tolist() == [4] * 8
    assert (ext.check_results_batch(st, 8) == 0).all()


@pytest.mark.parametrize("name", ["c1", "c2", "c3"])
def test_golden_moves_features(ext, oracle, name):
    g = load_golden(name)
    B = len(g["states"])
    st = _cuda(g["states"])
    moves, n = ext.generate_legal_moves_batch(st, B)
    assert np.array_equal(n.cpu().numpy(), g["n"])
    assert np.array_equal(moves.cpu().numpy(), g["moves"])
    moves2, n2, feat = ext.generate_legal_moves_and_fnn_features_batch(st, B)
    assert np.array_equal(moves2.cpu().numpy(), g["moves"])
    assert np.array_equal(_bits(feat.cpu().numpy()), _bits(g["features"]))
    feat2 = ext.extract_fnn_features_batch(st, _cuda(g["moves"]), _cuda(g["n"]), B)
    assert np.array_equal(_bits(feat2.cpu().numpy()), _bits(g["features"]))
    # compact successor lists of the golden moves, via extract on the oracle's compact lists
    feat3 = ext.extract_fnn_features_batch(st, _cuda(g["compact"]), _cuda(g["ncompact"]), B)
    want3 = np.stack([oracle.fnn_features(g["states"][i], g["compact"][i], int(g["ncompact"][i]))
                      for i in range(B)])
    assert np.array_equal(_bits(feat3.cpu().numpy()), _bits(want3))


@pytest.mark.parametrize("ordered", [True, False], ids=["turn-order", "index-order"])
@pytest.mark.parametrize("B", [1, 2, 3, 5, 7, 130])
def test_small_batches(ext, B, ordered):
    """Small and odd batch sizes, fused entry point against the golden lists."""
    g = load_golden("c3")
    st = _cuda(g["states"][1:B + 1])
    moves, n, feat, act = ext.generate_legal_moves_features_actions_batch(st, B, ordered=ordered)
    assert np.array_equal(n.cpu().numpy(), g["n"][1:B + 1])
    assert np.array_equal(moves.cpu().numpy(), g["moves"][1:B + 1])
    assert np.array_equal(_bits(feat.cpu().numpy()), _bits(g["features"][1:B + 1]))
    act2 = ext.legal_moves_to_actions_batch(st, moves, n, B)
    assert torch.equal(act, act2)


def test_turn_order_workspace_reuse(ext, oracle):
    """hg_legal_features_actions_ordered on one zero-filled workspace across
    calls of alternating parity (each call counts into one array and clears
    the other), with batches that shrink and grow: every call matches the
    index-order launch; a parity other than 0 / 1 is refused."""
    import ctypes
    lib = ext._lib
    states, _ = _oracle_positions(oracle, 4096, 7, 150, seed=0xACE)
    st = _cuda(states)
    ws = torch.zeros((int(lib.hg_legal_features_actions_ordered_workspace(4096)) // 4,), dtype=torch.int32,
                     device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for k, B in enumerate((4096, 1000, 4096, 3, 2048)):
        moves = torch.empty((B, 256, 6), dtype=torch.uint8, device="cuda")
        n = torch.empty((B,), dtype=torch.int32, device="cuda")
        feat = torch.empty((B, 122), dtype=torch.float32, device="cuda")
        act = torch.empty((B, 256), dtype=torch.int32, device="cuda")
        rc = lib.hg_legal_features_actions_ordered(st.data_ptr(), B, moves.data_ptr(), n.data_ptr(), feat.data_ptr(),
                                                   act.data_ptr(), ws.data_ptr(), k & 1, stream)
        assert rc == 0
        plain = ext.generate_legal_moves_features_actions_batch(st[:B], B, ordered=False)
        for a, b in zip((moves, n, feat, act), plain):
            assert torch.equal(a, b), (k, B)
    assert lib.hg_legal_features_actions_ordered(st.data_ptr(), 3, moves.data_ptr(), n.data_ptr(), feat.data_ptr(),
                                                 act.data_ptr(), ws.data_ptr(), 2, stream) != 0
    # the Python entry keeps its own workspace per (device, stream) across calls
    for B in (4096, 17, 4096):
        out = ext.generate_legal_moves_features_actions_batch(st[:B], B)
        plain = ext.generate_legal_moves_features_actions_batch(st[:B], B, ordered=False)
        for a, b in zip(out, plain):
            assert torch.equal(a, b), B


@pytest.mark.parametrize("name", ["c1", "c2", "c3"])
def test_golden_successors_queen_escape_apply(ext, name):
    g = load_golden(name)
    st = _cuda(g["states"])
    succ = ext.fnn_successor_features_batch(st, _cuda(g["moves"]), _cuda(g["succ_root"]), _cuda(g["succ_idx"]),
                                            len(g["succ_root"]))
    assert np.array_equal(_bits(succ.cpu().numpy()), _bits(g["succ_features"]))
    qe = ext.queen_escape_flags_batch(st, len(g["states"]))
    assert np.array_equal(qe.cpu().numpy(), g["queen_escape"])
    k = min(512, len(g["succ_root"]))
    roots, idx = g["succ_root"][:k], g["succ_idx"][:k]
    children = _cuda(g["states"][roots])
    ext.apply_moves_batch(children, _cuda(g["moves"][roots, idx]), k)
    assert np.array_equal(children.cpu().numpy(), g["child_states"][:k])
    res = ext.check_results_batch(children, k).cpu().numpy()
    assert np.array_equal(res, g["child_states"][:k, 3415].astype(np.int32))


def _oracle_positions(oracle, B, mask, max_ply, seed=0x5EED):
    return oracle.generate_positions(B, mask, max_ply, seed, threads=16)


@pytest.mark.parametrize("cfg", [("c2", 65536, 0, 120), ("c3", 65536, 7, 150)], ids=["C2", "C3"])
def test_full_size_parity(ext, oracle, cfg):
    _, B, mask, max_ply = cfg
    states, _ = _oracle_positions(oracle, B, mask, max_ply)
    om, on, of, oa = oracle.batch_legal_features_actions(states, threads=16)
    st = _cuda(states)
    moves, n, feat, act = ext.generate_legal_moves_features_actions_batch(st, B)
    assert np.array_equal(n.cpu().numpy(), on)
    assert np.array_equal(moves.cpu().numpy(), om)
    assert np.array_equal(_bits(feat.cpu().numpy()), _bits(of))
    assert np.array_equal(act.cpu().numpy(), oa)
    act2 = ext.legal_moves_to_actions_batch(st, moves, n, B)
    assert np.array_equal(act2.cpu().numpy(), oa)
    # the launch in index order (hg_legal_features_actions) writes the same bytes
    plain = ext.generate_legal_moves_features_actions_batch(st, B, ordered=False)
    for a, b in zip((moves, n, feat, act), plain):
        assert torch.equal(a, b)
    cen = ext.compute_centroids_batch(st, B).cpu().numpy()
    for i in range(0, B, 997):
        assert tuple(cen[i]) == oracle.centroid(states[i])
    qe = ext.queen_escape_flags_batch(st, B).cpu().numpy()
    assert np.array_equal(qe, oracle.batch_queen_escape(states, threads=16))


@pytest.mark.parametrize("mask,max_ply", [(0, 120), (7, 150)])
def test_successor_features_scale(ext, oracle, mask, max_ply):
    states, _ = _oracle_positions(oracle, 1024, mask, max_ply, seed=0xBEEF)
    om, on, _, _ = oracle.batch_legal_features_actions(states, threads=16)
    roots = np.repeat(np.arange(len(states)), on).astype(np.int64)
    idx = np.concatenate([np.arange(k) for k in on]).astype(np.int64)
    want = oracle.batch_successor_features(states, om, roots, idx, full_list=False, threads=16)
    got = ext.fnn_successor_features_batch(_cuda(states), _cuda(om), _cuda(roots), _cuda(idx), len(roots))
    assert np.array_equal(_bits(got.cpu().numpy()), _bits(want))


@pytest.mark.parametrize("mask,max_ply", [(0, 120), (7, 150)])
def test_gpu_generator_matches_oracle(oracle, mask, max_ply):
    from hive_neuralnet_amd.hive_gpu import random_positions
    B = 4096
    st, plies = random_positions(B, mask, max_ply, 0x5EED)
    ost, oplies = _oracle_positions(oracle, B, mask, max_ply)
    assert np.array_equal(plies.cpu().numpy(), oplies)
    assert np.array_equal(st.cpu().numpy(), ost)


def test_lockstep_selfplay_golden():
    from hive_neuralnet_amd.hive_gpu import random_positions
    g = load_golden("c4")
    G = len(g["finals"])
    st, plies = random_positions(G, 0, int(g["max_ply"]), int(g["seed"]), lockstep=True)
    assert np.array_equal(plies.cpu().numpy(), g["plies"])
    assert np.array_equal(st.cpu().numpy(), g["finals"])


def test_c4_full_lockstep(oracle):
    """C4 at its configuration: all 16,384 lockstep games of the base game
    from the empty board, up to 300 plies (Philox (seed, game, ply) move
    choice); every final state byte and every game's ply count equal the
    oracle's replay of the same games."""
    from hive_neuralnet_amd.hive_gpu import random_positions
    G, P, seed = 16384, 300, 0x5EED + 3
    st, plies = random_positions(G, 0, P, seed, lockstep=True)
    ost, oplies = oracle.lockstep_selfplay(G, 0, P, seed)
    assert np.array_equal(plies.cpu().numpy(), oplies)
    assert np.array_equal(st.cpu().numpy(), ost)
    decided = int((ost[:, 3415] != 0).sum())
    assert 0 < decided < G  # the run covers finished and unfinished games


def test_lockstep_expansion_pieces(oracle):
    """The one-launch random play with mosquito, ladybug and pillbug (throws
    move other pieces, mosquitoes climb): 2,048 lockstep games to 300 plies,
    every final state byte and ply count equal to the oracle's replay."""
    from hive_neuralnet_amd.hive_gpu import random_positions
    G, P, seed = 2048, 300, 0x5EED + 11
    st, plies = random_positions(G, 7, P, seed, lockstep=True)
    ost, oplies = oracle.lockstep_selfplay(G, 7, P, seed)
    assert np.array_equal(plies.cpu().numpy(), oplies)
    assert np.array_equal(st.cpu().numpy(), ost)
    assert 0 < int((ost[:, 3415] != 0).sum()) < G


def test_edge_cases(ext, oracle):
    e = ext.create_initial_states(0)
    m, n = ext.generate_legal_moves_batch(e, 0)
    assert m.shape == (0, 256, 6) and n.shape == (0,)
    # finished games: no moves, zero rows; features still defined
    g = load_golden("c4")
    done = g["finals"][g["finals"][:, 3415] != 0]
    assert len(done) > 0
    moves, n, feat = ext.generate_legal_moves_and_fnn_features_batch(_cuda(done), len(done))
    assert (n.cpu().numpy() == 0).all() and (moves.cpu().numpy() == 0).all()
    for i in range(len(done)):
        want = oracle.fnn_features(done[i], np.zeros((256, 6), np.uint8), 0)
        assert np.array_equal(_bits(feat[i].cpu().numpy()), _bits(want))
    # caller-supplied list longer than 256 is clamped; negative counts give none
    st = _cuda(g["finals"][:2])
    mv = torch.zeros((2, 256, 6), dtype=torch.uint8, device="cuda")
    f = ext.extract_fnn_features_batch(st, mv, torch.tensor([-3, 999], dtype=torch.int32, device="cuda"), 2)
    fin = g["finals"][:2]
    zeros = np.zeros((256, 6), np.uint8)
    want = np.stack([oracle.fnn_features(fin[0], zeros, 0), oracle.fnn_features(fin[1], zeros, 256)])
    assert np.array_equal(_bits(f.cpu().numpy()), _bits(want))


@pytest.mark.parametrize("T,zero_every", [(1, 0), (777, 0), (5000, 3)], ids=["one", "odd", "chunked-scan"])
def test_successor_rows_device_sized(ext, oracle, T, zero_every):
    """hg_successor_rows: offsets, total, row map and the successor features of
    every legal move, sized on the device, against the oracle.  T = 5,000
    leaves takes several legal counts per scan thread; every third leaf's
    count is forced to 0 (an idle row) there."""
    import ctypes
    st, _ = oracle.generate_positions(T, 7, 140, 0xABCD + T)
    moves, n, _, _ = oracle.batch_legal_features_actions(st, want_features=False, want_actions=False)
    n = n.astype(np.int32)
    if zero_every:
        n[::zero_every] = 0
    lib = ext._lib
    ws = torch.zeros((int(lib.hg_successor_rows_workspace(T)),), dtype=torch.uint8, device="cuda")
    feat = torch.full((T * 256, 122), float("nan"), dtype=torch.float32, device="cuda")
    s, m, nn = _cuda(st), _cuda(moves), _cuda(n)
    err = lib.hg_successor_rows(s.data_ptr(), m.data_ptr(), nn.data_ptr(), T, ws.data_ptr(), feat.data_ptr(),
                                torch.cuda.current_stream().cuda_stream)
    assert err == 0
    torch.cuda.synchronize()
    w = ws.view(torch.int64).cpu().numpy()
    offs, total = w[:T], int(w[T])
    want_offs = np.concatenate([[0], np.cumsum(n)[:-1]]).astype(np.int64)
    assert total == int(n.sum()) and np.array_equal(offs, want_offs)
    a2r, mi = w[T + 1: T + 1 + total], w[T + 1 + T * 256: T + 1 + T * 256 + total]
    want_a2r = np.repeat(np.arange(T), n).astype(np.int64)
    want_mi = np.concatenate([np.arange(k) for k in n]).astype(np.int64)
    assert np.array_equal(a2r, want_a2r) and np.array_equal(mi, want_mi)
    want = oracle.batch_successor_features(st, moves, want_a2r, want_mi)
    got = feat[:total].cpu().numpy()
    assert np.array_equal(_bits(got), _bits(want))


def test_successor_rows_large_batch(ext, oracle):
    """hg_successor_rows past the one-launch planner's batch limit (32,768
    leaves: there the offsets take one scan workgroup and the row map its own
    launch): 33,000 leaves, 1,000 positions tiled with every seventh count
    forced to 0.  Offsets, total and map in full; the features of the rows of
    the first and the last 300 leaves against the oracle."""
    T, P = 33000, 1000
    st1, _ = oracle.generate_positions(P, 7, 140, 0x5A5A)
    mv1, n1, _, _ = oracle.batch_legal_features_actions(st1, want_features=False, want_actions=False)
    st, moves = np.tile(st1, (T // P, 1)), np.tile(mv1, (T // P, 1, 1))
    n = np.tile(n1.astype(np.int32), T // P)
    n[::7] = 0
    lib = ext._lib
    ws = torch.zeros((int(lib.hg_successor_rows_workspace(T)),), dtype=torch.uint8, device="cuda")
    feat = torch.full((int(n.sum()), 122), float("nan"), dtype=torch.float32, device="cuda")
    s, m, nn = _cuda(st), _cuda(moves), _cuda(n)
    err = lib.hg_successor_rows(s.data_ptr(), m.data_ptr(), nn.data_ptr(), T, ws.data_ptr(), feat.data_ptr(),
                                torch.cuda.current_stream().cuda_stream)
    assert err == 0
    torch.cuda.synchronize()
    w = ws.view(torch.int64).cpu().numpy()
    offs, total = w[:T], int(w[T])
    want_offs = np.concatenate([[0], np.cumsum(n)[:-1]]).astype(np.int64)
    assert total == int(n.sum()) and np.array_equal(offs, want_offs)
    a2r, mi = w[T + 1: T + 1 + total], w[T + 1 + T * 256: T + 1 + T * 256 + total]
    want_a2r = np.repeat(np.arange(T), n).astype(np.int64)
    want_mi = np.concatenate([np.arange(k) for k in n]).astype(np.int64)
    assert np.array_equal(a2r, want_a2r) and np.array_equal(mi, want_mi)
    got = feat.cpu().numpy()
    for lo, hi in ((0, 300), (T - 300, T)):
        r0, r1 = int(want_offs[lo]), int(want_offs[hi - 1] + n[hi - 1])
        want = oracle.batch_successor_features(st, moves, want_a2r[r0:r1], want_mi[r0:r1])
        assert np.array_equal(_bits(got[r0:r1]), _bits(want))


def test_mismatched_shapes_rejected(ext):
    """A tensor whose trailing shape differs from the entry point's layout is
    rejected unless it is a flat contiguous buffer, which is taken as a view
    (so an output buffer is never silently replaced by a copy)."""
    st = ext.create_initial_states(4)
    with pytest.raises(ValueError, match="trailing shape"):
        ext.generate_legal_moves_batch(st.view(4, 214, 16), 4)
    with pytest.raises(ValueError, match="trailing shape"):
        ext.generate_legal_moves_batch(st.view(8, 1712), 4)
    flat = st.reshape(-1)
    m1, n1 = ext.generate_legal_moves_batch(flat, 4)
    m2, n2 = ext.generate_legal_moves_batch(st, 4)
    assert torch.equal(m1, m2) and torch.equal(n1, n2)
    # a flat out= buffer is written in place
    legal, nl = m2, n2
    a2r = torch.zeros((int(nl[0].item()),), dtype=torch.int64, device="cuda")
    mi = torch.arange(a2r.shape[0], dtype=torch.int64, device="cuda")
    want = ext.fnn_successor_features_batch(st, legal, a2r, mi, a2r.shape[0])
    out = torch.full((a2r.shape[0] * 122,), float("nan"), dtype=torch.float32, device="cuda")
    ext.fnn_successor_features_batch(st, legal, a2r, mi, a2r.shape[0], out=out)
    assert torch.equal(out.view(-1, 122), want)
    with pytest.raises(ValueError, match="trailing shape"):
        ext.fnn_successor_features_batch(st, legal, a2r, mi, a2r.shape[0], out=out.view(-1, 61))


@pytest.mark.parametrize("B,mask,P,lockstep", [(1, 0, 40, True), (777, 7, 90, True), (513, 0, 120, False),
                                               (300, 7, 150, False)])
def test_random_play_one_launch_equals_per_ply(B, mask, P, lockstep):
    """hg_random_play (every ply in one launch, workgroups keeping their games)
    against hg_random_play_step after each ply's legal lists: the same final
    rows and ply counts, odd batches (a workgroup with one game) included."""
    from hive_neuralnet_amd.hive_gpu import random_positions
    a = random_positions(B, mask, P, 0x5EED + 9, lockstep=lockstep, per_ply=False)
    b = random_positions(B, mask, P, 0x5EED + 9, lockstep=lockstep, per_ply=True)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_random_play_pair_counter_scratch(ext):
    """hg_random_play with more game pairs than the device holds at once
    (12,001 games: workgroups take the pairs beyond their first from the
    counter kept in the scratch), on a scratch pointer one byte past an
    aligned address, reused by a second, smaller call: the rows and ply
    counts of the per-ply launches both times."""
    import ctypes
    from hive_neuralnet_amd.hive_gpu import random_positions
    lib = ext._lib
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    scratch = torch.empty((12001 * 256 * 6 + 8,), dtype=torch.uint8, device="cuda")
    for B, P, lockstep in ((12001, 60, False), (999, 40, True)):
        seed = 0xC0DE + B
        want_states, want_plies = random_positions(B, 0, P, seed, lockstep=lockstep, per_ply=True)
        st = ext.create_initial_states(B, 0)
        plies = torch.zeros((B,), dtype=torch.int32, device="cuda")
        rc = lib.hg_random_play(st.data_ptr(), scratch.data_ptr() + 1, B, P, 1 if lockstep else 0, seed,
                                plies.data_ptr(), stream)
        assert rc == 0
        torch.cuda.synchronize()
        assert torch.equal(st, want_states) and torch.equal(plies, want_plies)
