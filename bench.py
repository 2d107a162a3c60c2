"""Benchmark of the batched Hive engine on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Workload ("C2"): 65,536 base-game positions from
seeded Philox random play (plies uniform in [0, 120]), resident in HBM.  One
step = one pass of the hot path over the batch: legal-move generation + the
122-dim FNN features + legal-move -> action-index lookup, through the fused
C-ABI entry point hg_legal_features_actions.  Prints one JSON line.

Roofline: the dominant (only) kernel is k_legal<moves,features,actions>;
algorithmic bytes per position = state 3424 + moves 1536 + n 4 + features
488 + actions 1024 = 6476 B.  `achieved` = 6476 B x batch / the step's GPU
time: one HIP event pair on the launch stream around K back-to-back calls of
the C-ABI entry (outputs allocated once), / K, median of 5 groups; beside it
the committed rocprof average of k_legal and the host cost per public call.

cpu_baseline: this repository's C restatement of the reference algorithm
(oracle/, "port", the same work: moves + features + action indices) on
every host CPU granted to the job, with nproc, the affinity mask, the cgroup
quota and the CPU model.  The reference's own CPU build never runs here.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

BYTES_PER_POSITION = 3424 + 256 * 6 + 4 + 122 * 4 + 256 * 4  # 6476
HBM_PEAK_GBS = 8000.0
C4_BYTES_PER_PLY = 2 * 3424  # lockstep random play, unfused model: the state read and written back
SEED = 0x5EED


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 100 steps of ~0.2 ms: a one-off host stall of the Python launcher is a
    # small part of the 20 ms timed region
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--batch", type=int, default=65536)
    ap.add_argument("--max-ply", type=int, default=120)
    ap.add_argument("--mask", type=int, default=0)
    ap.add_argument("--cpu-threads", type=int, default=0, help="0 = every CPU granted to the job")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="target CPU-thread seconds for the baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-mcts", action="store_true", help="skip the C5 Gumbel self-play leg")
    ap.add_argument("--mcts-only", action="store_true", help="run only the C5 leg (its own JSON line)")
    ap.add_argument("--c4-only", action="store_true", help="run only the C4 leg (its own JSON line)")
    ap.add_argument("--no-probe", action="store_true", help="skip the root tactical probe leg")
    ap.add_argument("--no-train", action="store_true", help="skip the training forward-batch leg")
    ap.add_argument("--no-c4", action="store_true", help="skip the C4 lockstep random-play leg")
    ap.add_argument("--no-c3", action="store_true", help="skip the C3 expansion-piece positions leg")
    ap.add_argument("--c4-games", type=int, default=16384)
    ap.add_argument("--c4-plies", type=int, default=300)
    ap.add_argument("--game-parts", type=int, default=None,
                    help="C5 game ranges whose waves run on their own streams (default: 2 from 256 games)")
    ap.add_argument("--mcts-waves", choices=("schedule", "1"), default="schedule",
                    help="C5 simulations per candidate per wave: the (2,4,8,16) schedule or 1")
    ap.add_argument("--mcts-games", type=int, default=512)
    ap.add_argument("--mcts-sims", type=int, default=4096)
    ap.add_argument("--mcts-plies", type=int, default=3, help="timed self-play plies")
    ap.add_argument("--mcts-warmup", type=int, default=1, help="untimed self-play plies before timing")
    ap.add_argument("--mcts-roots", choices=("empty", "midgame"), default="empty")
    ap.add_argument("--graphs", choices=("auto", "on", "off"), default="auto",
                    help="C5 simulation waves from HIP graphs: auto = waves under 2,048 rows")
    ap.add_argument("--ply-graphs", choices=("auto", "on", "off"), default="auto",
                    help="C5 search phase of a ply from one HIP graph: auto = when every round runs on one range")
    ap.add_argument("--native-waves", choices=("on", "off"), default="on",
                    help="C5 simulation waves as one library call each (on) or through the step entry points")
    ap.add_argument("--lib", default=None, metavar="PATH",
                    help="load this build of the engine instead of the package's own (a build-time alternative "
                         "made by `python -m hive_neuralnet_amd.build --define ... --out PATH`)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 256 MiB device-to-device copy 3 times (rocprof counter calibration)")
    return ap.parse_args()


def profile_figure(name, key):
    """A `key: value` figure from a committed profiles/ summary, else None."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    m = re.search(rf"^{key}:\s*([0-9.eE+]+)", open(path).read(), re.M)
    return float(m.group(1)) if m else None


def traffic_per_launch(config="C2"):
    """HBM bytes per launch of k_legal at a configuration, from the committed
    rocprofv3 --pmc summary (profiles/k_legal_<config>_traffic.txt), else None."""
    path = os.path.join(ROOT, "profiles", f"k_legal_{(config or '').lower()}_traffic.txt")
    if not config or not os.path.exists(path):
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", open(path).read())
    return float(m.group(1)) if m else None


def rocprof_kernel_us(config):
    """Average k_legal<true,true,true,true> duration (us) in the committed
    rocprofv3 --kernel-trace --stats summary for `config`, else None."""
    path = os.path.join(ROOT, "profiles", f"k_legal_{(config or '').lower()}_kernel_stats.md")
    if not config or not os.path.exists(path):
        return None
    m = re.search(r"^\| k_legal<true, true, true, true>[^|]*\|\s*\d+\s*\|\s*([0-9.]+)", open(path).read(), re.M)
    return float(m.group(1)) if m else None


def step_gpu_time(ext, states, B, K, groups=5):
    """Seconds of GPU time per fused turn-ordered step: per group, one HIP event
    pair on the launch stream around K back-to-back hg_legal_features_actions_ordered
    calls through the C-ABI with outputs and workspace allocated once (the host
    enqueues far faster than the kernels run, so the stream never idles between
    them), divided by K; the median of `groups` groups."""
    import torch

    lib = ext._lib
    moves = torch.empty((B, 256, 6), dtype=torch.uint8, device="cuda")
    n = torch.empty((B,), dtype=torch.int32, device="cuda")
    feat = torch.empty((B, 122), dtype=torch.float32, device="cuda")
    act = torch.empty((B, 256), dtype=torch.int32, device="cuda")
    ws = torch.zeros((int(lib.hg_legal_features_actions_ordered_workspace(B)) // 4,), dtype=torch.int32,
                     device="cuda")
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    args = (states.data_ptr(), B, moves.data_ptr(), n.data_ptr(), feat.data_ptr(), act.data_ptr(), ws.data_ptr())
    parity = 0

    def call():
        nonlocal parity
        err = lib.hg_legal_features_actions_ordered(*args, parity, sp)
        if err:
            raise RuntimeError(f"hg_legal_features_actions_ordered failed: {err}")
        parity ^= 1

    for _ in range(3):
        call()
    torch.cuda.synchronize()
    per = []
    for _ in range(groups):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(K):
            call()
        b.record(stream)
        torch.cuda.synchronize()
        per.append(a.elapsed_time(b) / 1e3 / K)
    return statistics.median(per)


def host_cpus():
    """The host CPUs this process may use: os.cpu_count() (nproc of the
    machine), the affinity mask, the cgroup CPU quota, and the thread count
    the CPU baselines use -- every CPU granted to the job (the smaller of the
    affinity mask and the quota).  With the full model name."""
    nproc = os.cpu_count() or 1
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = nproc
    quota = None
    try:
        q, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if q != "max":
            quota = float(q) / float(period)
    except (OSError, ValueError):
        pass
    threads = affinity if quota is None else max(1, min(affinity, int(quota + 0.5)))
    model = "unknown"
    try:
        model = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name"))
    except (OSError, StopIteration):
        pass
    return {"nproc": nproc, "affinity": affinity, "cgroup_quota": quota, "threads": threads, "cpu_model": model}


def baseline_threads(args):
    return args.cpu_threads or host_cpus()["threads"]


def cpu_baseline(states_np, threads, target_s):
    """The oracle's moves + features + action indices over the workload on
    `threads` pthreads, median of 5 passes; one thread over a slice beside it."""
    from oracle import Oracle
    orc = Oracle()
    B = states_np.shape[0]
    orc.batch_legal_features_actions(states_np[: min(B, 4096)], threads=threads)  # warm
    rates = []
    for _ in range(5):
        t0 = time.perf_counter()
        orc.batch_legal_features_actions(states_np, threads=threads)
        rates.append(B / (time.perf_counter() - t0))
    one = states_np[: min(B, 8192)]
    t0 = time.perf_counter()
    orc.batch_legal_features_actions(one, threads=1)
    per_core = one.shape[0] / (time.perf_counter() - t0)
    cpus = host_cpus()
    return {
        "value": statistics.median(rates), "unit": "positions/s", "cores": threads, "kind": "port",
        "sample": f"the full {B}-position workload, 5 passes, median; oracle/hive_oracle.c "
                  f"(moves + features + action indices), {threads} pthreads = every CPU granted to this job",
        "per_core_value": per_core, "per_core_sample": f"the first {one.shape[0]} positions on one thread",
        "nproc_linear_estimate": per_core * cpus["nproc"], **cpus,
    }


def cpu_player_baseline(net, roots_np, sims, threads):
    """The reference's CPU search player (FNNNativeCPUPlayer, fnn_native_cpu_player.py:126-266)
    restated in oracle/hive_cpu_player.c: per game a serial Gumbel search of `sims`
    simulations, each leaf evaluated with full-list successor features and the fp32
    network; one game per thread at a time, three games per thread from the timed
    ply's roots (about 20 thread-seconds from the empty board)."""
    import numpy as np
    from oracle import Oracle
    orc = Oracle()
    W = {k: v.detach().float().cpu().numpy() for k, v in net.state_dict().items()}
    live = roots_np[roots_np[:, 3415] == 0]
    sample = live[:3 * threads]
    t0 = time.perf_counter()
    _, done = orc.cpu_player_search(sample, W, sims, 16, threads=threads)
    wall = time.perf_counter() - t0
    return {
        "value": float(done.sum()) / wall, "unit": "sims/s", "cores": threads, "kind": "port",
        "sample": f"{sample.shape[0]} of the first timed ply's roots, one game per thread at a time, {sims} simulations "
                  "each: FNNNativeCPUPlayer's serial Gumbel search (full-list successor features, fp32 network) "
                  f"restated in oracle/hive_cpu_player.c; {int(done.sum())} simulations in {wall:.2f} s",
        **host_cpus(),
    }


def mcts_cpu_baseline(net, leaves_np, threads, target_s):
    """Leaf evaluation on the host: legal moves + root features + successor
    features of every legal move (oracle/hive_oracle.c, compact list as the GPU)
    + the FNN forward in numpy fp32.  Tree select/backup are left out (well
    under 1% of a simulation on the CPU), so this is an upper bound on CPU sims/s."""
    import numpy as np
    from oracle import Oracle
    orc = Oracle()
    W = {k: v.detach().float().cpu().numpy() for k, v in net.state_dict().items()}

    def lin(x, name):
        return x @ W[name + ".weight"].T + W[name + ".bias"]

    def encode(x):
        h = 1.0 / (1.0 + np.exp(-lin(x, "fc1")))
        mu = h.mean(axis=1, keepdims=True)
        var = ((h - mu) ** 2).mean(axis=1, keepdims=True)
        h = (h - mu) / np.sqrt(var + 1e-5) * W["ln1.weight"] + W["ln1.bias"]
        return lin(h, "fc2")

    def evaluate(states):
        moves, n, feat, _ = orc.batch_legal_features_actions(states, threads=threads, want_actions=False)
        a2r = np.repeat(np.arange(states.shape[0]), n).astype(np.int64)
        mi = np.concatenate([np.arange(k) for k in n]).astype(np.int64) if len(n) else np.zeros(0, np.int64)
        succ = orc.batch_successor_features(states, moves, a2r, mi, threads=threads)
        emb = encode(np.concatenate([feat, succ]).astype(np.float32))
        r, sc = emb[: states.shape[0]], emb[states.shape[0]:]
        np.tanh(lin(r, "value_fc"))
        np.tanh(lin(sc, "value_fc"))
        x = 1.0 / (1.0 + np.exp(-lin(np.concatenate([r[a2r], sc], axis=1), "action_fc1")))
        return lin(x, "action_fc2")

    L = leaves_np.shape[0]
    t0 = time.perf_counter()
    evaluate(leaves_np[: min(L, 512)])
    one = (time.perf_counter() - t0) / min(L, 512)
    count = int(max(256, min(L, target_s / max(one, 1e-9) / 3)))
    sample = leaves_np[:count]
    rates = []
    for _ in range(3):
        t0 = time.perf_counter()
        evaluate(sample)
        rates.append(count / (time.perf_counter() - t0))
    return {
        "value": statistics.median(rates), "unit": "sims/s", "cores": threads, "kind": "port",
        "sample": f"{count} leaf states from the GPU search's last wave, 3 passes, median; leaf evaluation only "
                  f"(legal list + features + successor features via oracle/hive_oracle.c with {threads} pthreads, "
                  "FNN large in numpy fp32)",
    }


def mcts_leg(args):
    """C5: Gumbel-root self-play over `--mcts-games` games with `--mcts-sims`
    simulations per move, k=16, FNN `large` random init (torch.manual_seed)."""
    import numpy as np
    import torch
    from hive_neuralnet_amd import hive_gpu
    from hive_neuralnet_amd.fnn import seeded_large
    from hive_neuralnet_amd.orchestrator import FNNMCTSConfig, FNNMCTSOrchestrator

    G, S = args.mcts_games, args.mcts_sims
    net = seeded_large(SEED)
    cfg = FNNMCTSConfig(num_simulations=S, max_num_considered_actions=16, batch_size=G,
                        max_tree_nodes=1 + S * 256, wave_parallel=args.mcts_waves == "schedule")
    orch = FNNMCTSOrchestrator(net, cfg)
    orch.use_graphs = {"auto": None, "on": True, "off": False}[args.graphs]
    orch.use_ply_graphs = {"auto": None, "on": True, "off": False}[args.ply_graphs]
    orch.game_parts = args.game_parts
    orch.native_waves = args.native_waves == "on"
    ext = orch.ext
    if args.mcts_roots == "empty":
        states = ext.create_initial_states(G, 0)
    else:
        states, _ = hive_gpu.random_positions(G, 0, 120, SEED)
    torch.manual_seed(SEED + 1)
    np.random.seed(SEED & 0xFFFF)
    tree = orch._alloc_tree(G)
    active = torch.ones((G,), dtype=torch.bool, device="cuda")

    def ply():
        r = orch.search_ply(states, tree, active)
        orch.apply_and_rebase(states, tree, r)
        active.logical_and_(ext.check_results_batch(states, G) == 0)

    # counters first: their address is part of a captured ply graph's key, so the
    # warm-up ply captures the graph the timed plies replay
    orch.enable_counters()
    for _ in range(args.mcts_warmup):
        ply()
    timed_roots = states.clone()  # the first timed ply's roots (the CPU player searches the same positions)
    orch._stats.zero_()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.mcts_plies):
        ply()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    c = {k: int(v.item()) for k, v in orch.counters.items()}
    sims = c["sims"]
    Lm = c["leaf_legal"] / max(1, sims)
    Dm = c["vl_len"] / max(1, sims)
    b_sim = 5976 + 535 * Lm + 16 * Dm
    value = sims / wall
    achieved = b_sim * value / 1e9
    out = {
        "metric": "MCTS sims/sec at 512 games", "value": value, "unit": "sims/s", "plies": args.mcts_plies,
        "warmup_plies": args.mcts_warmup, "ms_per_ply": wall / args.mcts_plies * 1e3,
        "config": {"workload": f"C5: Gumbel-root self-play, {G} games from the "
                               f"{'empty board' if args.mcts_roots == 'empty' else 'C2-style mid-game roots'}, "
                               f"{S} sims/move, k=16, "
                               f"{'wave schedule (2,4,8,16)' if cfg.wave_parallel else 'one simulation per candidate per wave'}, "
                               "FNN large random init",
                   "games": G, "sims_per_move": S, "max_tree_nodes": 1 + S * 256, "seed": SEED,
                   "roots": args.mcts_roots},
        "simulations": sims, "sim_rows": c["rows"], "mean_leaf_legal": Lm, "mean_vl_len": Dm,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS,
                     "traffic": (profile_figure("mcts_c5_traffic.txt", "traffic_bytes_per_sim")
                                 if args.mcts_roots == "empty" and cfg.wave_parallel else None),
                     "traffic_is": "HBM bytes per simulation over the schedule's waves from the empty board, "
                                   "rocprofv3 FETCH_SIZE + WRITE_SIZE (profiles/mcts_c5_traffic.txt)",
                     "bytes_per_sim": b_sim, "formula": "5976 + 535*L + 16*D"},
    }
    if not args.no_cpu:
        threads = baseline_threads(args)
        out["cpu_baseline"] = cpu_player_baseline(net, timed_roots.cpu().numpy(), S, threads)
        out["gpu_over_cpu"] = value / out["cpu_baseline"]["value"]
        orch.keep_last_leaves = True
        orch.counters = None
        cfg.num_simulations = min(S, 256)
        orch.search_ply(states, tree, active)
        leaves = orch.last_leaves.cpu().numpy()
        out["cpu_leaf_eval_bound"] = mcts_cpu_baseline(net, leaves, threads, args.cpu_seconds)
    return out


def probe_leg(args):
    """Root tactical probe (root_tactical_probe_batch, the trainer's default root
    analysis) on 4,096 seeded random-play positions (plies U[0,150]), every
    stage enabled; the oracle on the host cores beside it."""
    import numpy as np
    import torch
    from hive_neuralnet_amd import hive_gpu
    ext = hive_gpu.load_extension()
    B = 4096
    states, _ = hive_gpu.random_positions(B, 0, 150, SEED + 7)
    legal, nl = ext.generate_legal_moves_batch(states, B)
    pr = torch.from_numpy((np.random.default_rng(SEED).integers(0, 8, size=(B, 256)) / 8.0).astype(np.float32)).cuda()
    for _ in range(2):
        ext.root_tactical_probe_batch(states, legal, nl, pr, B)
    torch.cuda.synchronize()
    reps = 5
    t0 = time.perf_counter()
    for _ in range(reps):
        w, a, f = ext.root_tactical_probe_batch(states, legal, nl, pr, B)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / reps * 1e3
    out = {"metric": "root tactical probes/s", "value": B / ms * 1e3, "unit": "roots/s", "ms_per_call": ms,
           "config": {"workload": "4,096 base-game positions, plies U[0,150], all probe stages", "batch": B},
           "immediate_or_forced_wins": int((w >= 0).sum().item()), "forced_random": int(f.sum().item())}
    if not args.no_cpu:
        from oracle import Oracle
        threads = baseline_threads(args)
        st, lm, n, p = states.cpu().numpy(), legal.cpu().numpy(), nl.cpu().numpy(), pr.cpu().numpy()
        orc = Oracle()
        t0 = time.perf_counter()
        orc.batch_root_tactical_probe(st, lm, n, p, threads=threads)
        dt = time.perf_counter() - t0
        out["cpu_baseline"] = {"value": B / dt, "unit": "roots/s", "cores": threads, "kind": "port",
                               "sample": f"the same {B} roots, oracle/hive_oracle.c, {threads} pthreads, one pass"}
    return out


def train_leg(args):
    """Training-time encoder path (FNNTrainer._build_forward_batch counterpart):
    roots + every legal successor's features for a 2,048-position batch drawn
    from C2-style positions, uncached (legal lists + features generated)."""
    import torch
    from hive_neuralnet_amd import hive_gpu
    from hive_neuralnet_amd.replay import build_forward_batch
    ext = hive_gpu.load_extension()
    B = 2048
    states, _ = hive_gpu.random_positions(B, 0, 120, SEED + 11)
    for _ in range(2):
        build_forward_batch(ext, states, B)
    torch.cuda.synchronize()
    reps = 10
    t0 = time.perf_counter()
    for _ in range(reps):
        _, succ, _, _ = build_forward_batch(ext, states, B)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / reps * 1e3
    return {"metric": "training forward batches/s", "value": 1e3 / ms, "unit": "batches/s", "ms_per_batch": ms,
            "positions_per_s": B / ms * 1e3, "successor_rows_per_s": succ.shape[0] / ms * 1e3,
            "config": {"workload": "2,048 base-game positions (plies U[0,120]) + all legal successors, uncached",
                       "batch": B, "successor_rows": int(succ.shape[0])}}


def fnv1a64_rows(states_np):
    """FNV-1a-64 of each state row, padding bytes 3174-3175 and 3420-3423
    masked to zero (they carry no state)."""
    import numpy as np
    x = states_np.copy()
    x[:, 3174:3176] = 0
    x[:, 3420:3424] = 0
    h = np.full(x.shape[0], 0xCBF29CE484222325, dtype=np.uint64)
    prime = np.uint64(0x100000001B3)
    with np.errstate(over="ignore"):
        for j in range(x.shape[1]):
            h ^= x[:, j].astype(np.uint64)
            h *= prime
    return h


def fnv1a64_of(hashes):
    """FNV-1a-64 over the little-endian bytes of a hash list."""
    import numpy as np
    return int(fnv1a64_rows(hashes.astype("<u8").view(np.uint8).reshape(1, -1))[0])


def c4_leg(args):
    """C4: 16,384 lockstep random games from the empty board, up to 300 plies,
    Philox (seed, game, ply) move choice; every ply one legal-move generation
    over all games and one move step (finished games stay put)."""
    import numpy as np
    import torch
    from hive_neuralnet_amd import hive_gpu
    G, P = args.c4_games, args.c4_plies
    hive_gpu.random_positions(256, 0, 8, SEED + 3, lockstep=True)  # warm
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    states, plies = hive_gpu.random_positions(G, 0, P, SEED + 3, lockstep=True)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    done = int(plies.sum().item())
    finals = states.cpu().numpy()
    hashes = fnv1a64_rows(finals)
    results = finals[:, 3415]
    out = {"metric": "lockstep random-play plies/s", "value": done / wall, "unit": "plies/s", "ms": wall * 1e3,
           "config": {"workload": f"C4: {G} lockstep games, base game, up to {P} plies, Philox (seed, game, ply)",
                      "games": G, "max_plies": P, "seed": SEED + 3},
           "plies_played": done, "games_decided": int((results != 0).sum()),
           "roofline": {"bound": "hbm", "achieved": done * C4_BYTES_PER_PLY / wall / 1e9, "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": done * C4_BYTES_PER_PLY / wall / 1e9 / HBM_PEAK_GBS,
                        "traffic": profile_figure("c4_traffic.txt", "traffic_bytes_per_ply"),
                        "traffic_is": "HBM bytes per played ply, from rocprofv3 FETCH_SIZE + WRITE_SIZE "
                                      "(profiles/c4_traffic.txt)",
                        "bytes_per_ply": C4_BYTES_PER_PLY, "model": "unfused: state read + write-back per ply"},
           "final_state_hash": f"{fnv1a64_of(hashes):016x}"}
    if not args.no_cpu:
        from oracle import Oracle
        threads = baseline_threads(args)
        orc = Oracle()
        k = min(G, 64)
        t1 = time.perf_counter()
        orc.lockstep_selfplay(k, 0, P, SEED + 3, threads=threads)
        one = (time.perf_counter() - t1) / k
        k = int(max(64, min(G, args.cpu_seconds / max(one * threads, 1e-9))))  # ~cpu_seconds of thread time
        t1 = time.perf_counter()
        cst, cpl = orc.lockstep_selfplay(k, 0, P, SEED + 3, threads=threads)
        cw = time.perf_counter() - t1
        out["cpu_baseline"] = {
            "value": int(cpl.sum()) / cw, "unit": "plies/s", "cores": threads, "kind": "port",
            "sample": f"the first {k} of the {G} games replayed by oracle/hive_oracle.c ({threads} pthreads)",
            "final_states_match": bool(np.array_equal(fnv1a64_rows(cst), hashes[:k])
                                       and np.array_equal(cpl, plies[:k].cpu().numpy())),
        }
    return out


def positions_leg(args, B, mask, max_ply):
    """One configuration of batched move generation + features + action indices
    (hg_legal_features_actions_ordered: k_order_buckets, then
    k_legal<true,true,true,true>) over B seeded
    random-play positions resident in HBM: positions/s over `steps` launches back
    to back, the kernel's mean time from HIP events, its HBM roofline, and the
    oracle on the host CPUs beside it."""
    import torch
    from hive_neuralnet_amd import hive_gpu

    ext = hive_gpu.load_extension()
    states, plies = hive_gpu.random_positions(B, mask, max_ply, SEED)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()

    def step():
        return ext.generate_legal_moves_features_actions_batch(states, B)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # the timed region: K launches back to back
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out = step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # host cost of one call of the public entry point: K enqueues with no wait
    # between them (the GPU runs behind; the loop ends when the last call returns)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(args.steps):
        step()
    host_ms_per_call = (time.perf_counter() - t1) / args.steps * 1e3
    torch.cuda.synchronize()
    step_gpu_s = step_gpu_time(ext, states, B, args.steps)
    moves, n, feat, act = out
    n_mean = float(n.float().mean().item())

    # unfused reference-API sequence, for comparison (not the headline)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    reps = max(1, args.steps // 2)
    for _ in range(reps):
        m2, n2, f2 = ext.generate_legal_moves_and_fnn_features_batch(states, B)
        ext.legal_moves_to_actions_batch(states, m2, n2, B)
    torch.cuda.synchronize()
    unfused = B * reps / (time.perf_counter() - t1)

    value = B * args.steps / wall
    achieved_gbs = BYTES_PER_POSITION * B / step_gpu_s / 1e9
    name = {(65536, 0, 120): "C2", (65536, 7, 150): "C3"}.get((B, mask, max_ply))
    ms_per_step = wall / args.steps * 1e3
    if step_gpu_s * 1e3 > ms_per_step * 1.001:
        print(f"bench: the step's GPU time {step_gpu_s * 1e3:.4f} ms exceeds the timed region's "
              f"{ms_per_step:.4f} ms per step", file=sys.stderr)
    rocprof_us = rocprof_kernel_us(name)
    out = {
        "value": value, "unit": "positions/s", "ms_per_step": ms_per_step,
        "config": {
            "workload": (f"{name}: fused legal moves + FNN features + action indices over {B:,} "
                         f"{'base-game' if mask == 0 else 'expansion-piece (mosquito, ladybug, pillbug)'} "
                         f"positions (plies U[0,{max_ply}])") if name else
                        f"batch {B}, expansion mask {mask}, plies U[0,{max_ply}]",
            "batch": B, "expansion_mask": mask, "max_ply": max_ply, "seed": SEED,
            "mean_legal_moves": n_mean, "mean_plies": float(plies.float().mean().item()),
            "entry_point": "hg_legal_features_actions_ordered",
        },
        "roofline": {
            "bound": "hbm", "achieved": achieved_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": achieved_gbs / HBM_PEAK_GBS, "traffic": traffic_per_launch(name),
            "kernel": "k_legal<true,true,true,true> (after k_order_buckets: the turn order)",
            "step_gpu_ms": step_gpu_s * 1e3,
            "step_gpu_ms_is": ("GPU time of one step (k_order_buckets + k_legal and the gap between them): "
                               "one HIP event pair on the launch stream around K back-to-back calls of the "
                               "C-ABI entry with preallocated outputs, / K; median of 5 such groups"),
            "step_gpu_within_ms_per_step": step_gpu_s * 1e3 <= ms_per_step * 1.001,
            "rocprof_k_legal_avg_us": rocprof_us,
            "frac_from_rocprof_avg": (BYTES_PER_POSITION * B / (rocprof_us * 1e-6) / 1e9 / HBM_PEAK_GBS
                                      if rocprof_us else None),
            "host_ms_per_call": host_ms_per_call,
            "bytes_per_position": BYTES_PER_POSITION,
        },
        "api_unfused_positions_per_s": unfused,
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(states.cpu().numpy(), baseline_threads(args), args.cpu_seconds)
        out["gpu_over_cpu"] = value / out["cpu_baseline"]["value"]
    return out


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}): positions and games are "
              "independent, so N GPUs shard the batch with no collectives; run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch

    if args.lib:
        from hive_neuralnet_amd import hive_gpu

        hive_gpu.load_library(os.path.abspath(args.lib))
    if args.copy_calibration:
        a = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": a.numel() * 4, "copies": 3}))
        return

    if args.mcts_only:
        print(json.dumps(mcts_leg(args)))
        return
    if args.c4_only:
        print(json.dumps(c4_leg(args)))
        return

    result = positions_leg(args, args.batch, args.mask, args.max_ply)
    result = {
        "metric": "positions/sec (move-gen+encode) at 65,536 batch; MCTS sims/sec at 512 games",
        "value": result.pop("value"),
        "unit": "positions/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": result.pop("ms_per_step"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int32",
        "data": "synthetic (seeded Philox random-play positions generated on the GPU)",
        **result,
    }
    if args.lib:
        result["lib"] = args.lib
    if not args.no_c3:  # configs[2]: the expansion-piece variant, same kernel and bytes per position
        c3 = positions_leg(args, 65536, 7, 150)
        c3["metric"] = "positions/sec (move-gen+encode), expansion pieces"
        result["c3"] = c3
    if not args.no_mcts:
        result["mcts"] = mcts_leg(args)
        mid = argparse.Namespace(**{**vars(args), "mcts_roots": "midgame", "no_cpu": args.no_cpu})
        result["mcts_midgame"] = mcts_leg(mid)
        if args.mcts_waves == "schedule":  # the second C5 schedule: one simulation per candidate per wave
            w1 = argparse.Namespace(**{**vars(args), "mcts_waves": "1", "no_cpu": True})
            result["mcts_w1"] = mcts_leg(w1)
    if not args.no_probe:
        result["probe"] = probe_leg(args)
    if not args.no_train:
        result["train"] = train_leg(args)
    if not args.no_c4:
        result["c4"] = c4_leg(args)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
