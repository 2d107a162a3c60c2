"""Benchmark of the batched Hive engine on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Workload ("C2"): 65,536 base-game positions from
seeded Philox random play (plies uniform in [0, 120]), resident in HBM.  One
step = one pass of the hot path over the batch: legal-move generation + the
122-dim FNN features + legal-move -> action-index lookup, through the fused
C-ABI entry point hg_legal_features_actions.  Prints one JSON line.

Roofline: the dominant (only) kernel is k_legal<moves,features,actions>;
algorithmic bytes per position = state 3424 + moves 1536 + n 4 + features
488 + actions 1024 = 6476 B.  `achieved` = 6476 B x batch / mean kernel
time measured with HIP events on the launch stream.

cpu_baseline: this repository's C restatement of the reference algorithm
(oracle/, "port", the same work: moves + features + action indices) on the
host cores; when oracle/_ref/libhive_ref.so (the reference's own CPU build)
is present, its legal-moves + features rate is reported beside it.
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
SEED = 0x5EED
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "k_legal_c2_traffic.txt")


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=65536)
    ap.add_argument("--max-ply", type=int, default=120)
    ap.add_argument("--mask", type=int, default=0)
    ap.add_argument("--cpu-threads", type=int, default=0, help="0 = min(16, cores)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="target CPU-thread seconds for the baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 256 MiB device-to-device copy 3 times (rocprof counter calibration)")
    return ap.parse_args()


def traffic_per_launch():
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, else None."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", open(TRAFFIC_FILE).read())
    return float(m.group(1)) if m else None


def cpu_baseline(states_np, threads, target_s):
    from oracle import Oracle, Reference
    orc = Oracle()
    B = states_np.shape[0]
    orc.batch_legal_features_actions(states_np[: min(B, 4096)], threads=threads)  # warm
    t0 = time.perf_counter()
    orc.batch_legal_features_actions(states_np, threads=threads)
    one = time.perf_counter() - t0
    reps = max(3, min(50, int(target_s / max(one * threads, 1e-6))))
    rates = []
    for _ in range(reps):
        t0 = time.perf_counter()
        orc.batch_legal_features_actions(states_np, threads=threads)
        rates.append(B / (time.perf_counter() - t0))
    out = {
        "value": statistics.median(rates), "unit": "positions/s", "cores": threads, "kind": "port",
        "sample": f"the full {B}-position workload, {reps} passes, median; oracle/hive_oracle.c "
                  f"(moves + features + action indices), {threads} pthreads",
    }
    ref = Reference.load()
    if ref is not None:
        ref.batch_legal_features(states_np[: min(B, 4096)], threads=threads)
        rr = []
        for _ in range(max(3, reps // 2)):
            t0 = time.perf_counter()
            ref.batch_legal_features(states_np, threads=threads)
            rr.append(B / (time.perf_counter() - t0))
        out["reference_value"] = statistics.median(rr)
        out["reference_sample"] = ("reference hive_gpu/csrc headers compiled for the host (oracle/_ref), "
                                   f"legal moves + features only, {threads} threads, same positions")
    try:
        out["cpu_model"] = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name"))
    except Exception:
        pass
    return out


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}): positions and games are "
              "independent, so N GPUs shard the batch with no collectives; run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch

    if args.copy_calibration:
        a = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": a.numel() * 4, "copies": 3}))
        return

    from hive_neuralnet_amd import hive_gpu

    ext = hive_gpu.load_extension()
    B = args.batch
    states, plies = hive_gpu.random_positions(B, args.mask, args.max_ply, SEED)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()

    def step():
        return ext.generate_legal_moves_features_actions_batch(states, B)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    t0 = time.perf_counter()
    for k in range(args.steps):
        starts[k].record(stream)
        out = step()
        ends[k].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kernel_ms = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    mean_kernel_s = statistics.mean(kernel_ms) / 1e3
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
    achieved_gbs = BYTES_PER_POSITION * B / mean_kernel_s / 1e9
    traffic = traffic_per_launch()
    result = {
        "metric": "positions/sec (move-gen+encode) at 65,536 batch; MCTS sims/sec at 512 games",
        "value": value,
        "unit": "positions/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall / args.steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int32",
        "data": "synthetic (seeded Philox random-play positions generated on the GPU)",
        "config": {
            "workload": "C2: fused legal moves + FNN features + action indices over 65,536 base-game positions "
                        "(plies U[0,120])" if (B == 65536 and args.mask == 0 and args.max_ply == 120) else
                        f"batch {B}, expansion mask {args.mask}, plies U[0,{args.max_ply}]",
            "batch": B, "expansion_mask": args.mask, "max_ply": args.max_ply, "seed": SEED,
            "mean_legal_moves": n_mean, "mean_plies": float(plies.float().mean().item()),
            "entry_point": "hg_legal_features_actions",
        },
        "roofline": {
            "bound": "hbm", "achieved": achieved_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": achieved_gbs / HBM_PEAK_GBS, "traffic": traffic,
            "kernel": "k_legal<true,true,true>", "mean_kernel_ms": mean_kernel_s * 1e3,
            "bytes_per_position": BYTES_PER_POSITION,
        },
        "api_unfused_positions_per_s": unfused,
    }
    if not args.no_cpu:
        threads = args.cpu_threads or max(1, min(16, os.cpu_count() or 1))
        result["cpu_baseline"] = cpu_baseline(states.cpu().numpy(), threads, args.cpu_seconds)
        result["gpu_over_cpu"] = value / result["cpu_baseline"]["value"]
    print(json.dumps(result))


if __name__ == "__main__":
    main()
