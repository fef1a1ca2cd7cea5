"""Benchmark: positions/s of the inference pass on one MI355X.

A step is one forward pass of the network over one batch of synthetic
positions already resident in HBM (the pass replayed as its captured
hipGraph). At 19x19 and 128 filters a batch that fills its rounds of one
workgroup per CU, the headline one included, runs the stem and the tower
as one launch with each board resident in a workgroup; other large
batches run as two half-batch chains on the slot's two streams, forked and
joined inside the graph. Default workload: 19x19, 10 residual blocks of 128
filters, batch 256 (the headline configuration). Prints one JSON line:
throughput, the dominant kernel's roofline (the board-resident launch, or
the residual-tower 3x3 convolution's launch over the whole batch, timed
live with HIP events on its stream, and beside it the tower's effective
time per layer as the pass runs it), and the CPU
baseline (the oracle's single-threaded blas pass, one worker per host core
at batch 8, as the reference bench's "cpu (blas)" row).

  python bench.py [--steps K] [--warmup W] [--workload 3] [--no-cpu] [--no-positions]

Three more modes serve the committed profiles (each prints one line):

  python bench.py --mode copy-calibration [--mib 256] [--conv-iters 5]
      a plain device-to-device copy of known size, for scaling rocprofv3's
      FETCH_SIZE / WRITE_SIZE readings to bytes;
  python bench.py --mode mfma-calibration [--conv-iters 5]
      dependent MFMA chains on every SIMD with nothing else in the way: the
      fp32 matrix rate the chip holds, beside the published peak;
  python bench.py --mode stem-heads [--workload 3] [--batch B] [--conv-iters 10]
      whole-batch launches of the stem convolution and the heads on one
      stream (in a pass of a large batch they run as two concurrent
      half-batch launches, whose traced durations overlap each other), for
      rocprofv3 --kernel-trace.

Beside the headline, "positions" times the steps either side of the pass
(azh_evaluate_positions: encoding from stone bytes, the legal moves with
superko, the priors) on the same boards, each position carrying 200
superko hashes, with the oracle's CPU restatement of the same two steps
timed on the host's cores (one worker per CPU, as the pass's baseline).

Runs on one GPU only: --gpus above 1 exits with a message.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "alphazero-go_amd")
sys.path.insert(0, PKG)

PEAK_FP32_MFMA_TFLOPS = 157.3     # MI355X dense fp32 matrix peak
PEAK_HBM_GBS = 8000.0
# The reference's published rate for this metric: CUDA fused kernels, 19x19
# 10x128 batch 256, 2 slots kept full, RTX 4070 Ti SUPER
# (docs/results/cuda-bench.txt:290).
REFERENCE_POS_PER_S = 6724.0


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", type=int, default=3, choices=[1, 2, 3, 4, 5])
    ap.add_argument("--batch", type=int, default=0, help="override the workload's batch")
    ap.add_argument("--conv-iters", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-calls", type=int, default=96, help="batch-8 passes per CPU worker")
    ap.add_argument("--no-positions", action="store_true", help="skip the positions path")
    ap.add_argument("--no-two-slot", action="store_true",
                    help="skip the runner-kept-full rate (its two slots overlap kernels; for kernel-trace profiles)")
    ap.add_argument("--seen", type=int, default=200, help="superko hashes per position")
    ap.add_argument("--mode", default="pass", choices=["pass", "copy-calibration", "mfma-calibration", "stem-heads"])
    ap.add_argument("--mib", type=int, default=256, help="copy-calibration: MiB copied per launch")
    return ap.parse_args()


# The committed rocprofv3 counter summaries, per dominant kernel.
TRAFFIC_PROFILES = {
    "conv3x3Tower": "conv3x3_tower_19x19_b256_hbm_traffic.txt",
    "convTowerResident": "resident_tower_19x19_b256_hbm_traffic.txt",
}


def traffic_from_profile(workload_name, kernel_hash, kernel):
    """HBM bytes per launch of the dominant kernel, from the committed
    rocprofv3 counter summary of the same kernel and sources, or None."""
    if kernel not in TRAFFIC_PROFILES:
        return None
    path = os.path.join(ROOT, "profiles", TRAFFIC_PROFILES[kernel])
    if not os.path.exists(path):
        return None
    vals = {}
    with open(path) as f:
        for line in f:
            if ":" in line and not line.startswith("#"):
                k, v = line.split(":", 1)
                vals[k.strip()] = v.strip()
    if vals.get("kernels") != kernel_hash or vals.get("workload") != workload_name or vals.get("kernel") != kernel:
        return None
    try:
        return float(vals["hbm_bytes_per_launch"])
    except (KeyError, ValueError):
        return None


def host_cpus():
    """The host's CPUs as this process sees them: the affinity set, the
    machine's count, and the container's CPU quota (cgroup v2 cpu.max) when
    one is set."""
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, period = f.read().split()
            if q != "max":
                quota = int(q) / int(period)
    except (OSError, ValueError):
        pass
    return {"affinity": affinity, "cpu_count": os.cpu_count(), "cgroup_quota": quota}


def cpu_workers():
    """One CPU-baseline worker per CPU this process may run on (its affinity
    set, within the container's CPU quota), and the host's counts."""
    host = host_cpus()
    workers = host["affinity"]
    if host["cgroup_quota"]:
        workers = max(1, min(workers, int(host["cgroup_quota"])))
    return workers, host


def cpu_baseline(workload, calls):
    """The oracle's blas pass (im2col + single-threaded OpenBLAS sgemm, the
    reference's CPU backend restated) on this host: one worker per CPU the
    process may run on (the affinity set, within the container's CPU quota),
    each running `calls` passes of batch 8 (the reference bench's "cpu
    (blas)" row, apps/bench.cpp:452-476), plus one batch-256 pass on one
    worker."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    w = O.WORKLOADS[workload]
    net = O.init_network(w.cfg)
    workers, host = cpu_workers()
    inp8, _ = O.workload_inputs(w, 8)
    rate, elapsed = O.time_workers(net, inp8, workers, calls, O.BLAS)
    one_b = min(w.batch, 256)
    inp_one, _ = O.workload_inputs(w, one_b)
    rate_one, el_one = O.time_workers(net, inp_one, 1, 1, O.BLAS, warm=False)
    return {
        "value": round(rate, 2),
        "unit": "positions/s",
        "cores": workers,
        "host_cpus": host,
        "kind": "port",
        "sample": f"{workers} single-threaded workers (one per host CPU) x {calls} passes of batch 8 "
                  f"({workers * calls * 8} positions, {elapsed:.1f} s); oracle blas restatement of Network::infer",
        "single_worker_batch": one_b,
        "single_worker_seconds": round(el_one, 2),
        "single_worker_value": round(rate_one, 2),
        "blas": O.blas_description(),
    }


def copy_calibration(mib, iters):
    """A plain device copy of known size: FETCH_SIZE and WRITE_SIZE per
    dispatch against the bytes moved give the counters' scale factors."""
    import azgo_hip
    nbytes = mib << 20
    ms = azgo_hip.probe_copy(nbytes, iters)
    print(json.dumps({"mode": "copy-calibration", "bytes_per_copy": nbytes, "copies": iters,
                      "ms_per_copy": round(ms / iters, 4),
                      "gb_s_read_plus_write": round(2 * nbytes / (ms / iters * 1e-3) / 1e9, 1)}), flush=True)


def mfma_calibration(iters):
    """The fp32 matrix units' rate with nothing else in the way: one 8-wave
    workgroup per CU, each wave a dependent chain of 80,000 16x16x4 MFMAs
    (two waves per SIMD, so each SIMD alternates between two chains and
    issues one MFMA every 32 cycles): the clock the chip holds under a full
    MFMA load, against the 2.4 GHz of the published peak."""
    import azgo_hip
    ms, flops = azgo_hip.probe_mfma(20000, iters)
    tf = flops / (ms / iters * 1e-3) / 1e12
    print(json.dumps({"mode": "mfma-calibration", "launches": iters, "ms_per_launch": round(ms / iters, 4),
                      "flops_per_launch": flops, "tflops": round(tf, 2),
                      "frac_of_published_peak": round(tf / PEAK_FP32_MFMA_TFLOPS, 4),
                      "implied_clock_ghz": round(2.4 * tf / PEAK_FP32_MFMA_TFLOPS, 3)}), flush=True)


def stem_heads(workload, B, iters):
    """Whole-batch launches of the heads (on a trunk uploaded before each)
    and of the stem convolution (the input planes to F channels, the
    batch's workgroup shape) on one stream, random weights with BN
    variances in [0.5, 1.5]."""
    import numpy as np
    import azgo_hip
    import workload as W
    w = W.WORKLOADS[workload]
    B = B or w.batch
    n, H, blocks, F, V = w.cfg
    cfg = azgo_hip.net_cfg(n, H, blocks, F, V)
    rng = np.random.default_rng(1)
    tensors = {name: rng.uniform(*((0.5, 1.5) if name.endswith("runVar") else (-0.05, 0.05)), floats)
               .astype(np.float32) for name, floats in azgo_hip.tensor_spec(cfg)}
    with azgo_hip.Runner(cfg, tensors, B, 1) as r:
        trunk = rng.uniform(0, 2, (B, F, n * n)).astype(np.float32)
        for _ in range(iters):
            r.probe_heads(trunk)
    ms = azgo_hip.time_conv3x3(B, n, cfg.planes, F, -1, iters)   # average per launch
    print(json.dumps({"mode": "stem-heads", "workload": f"{n}x{n} {blocks}x{F} batch {B}", "head_launches": iters,
                      "stem_us_per_launch": round(ms * 1e3, 2)}), flush=True)


def positions_leg(r, w, B, seen_per_position, iters=20, passes=None):
    """The positions path on the benchmark's boards (no history: ply 0 only),
    device-resident: HIP events around each step (encode, legal moves,
    priors) and the whole chain (encode, pass, legal moves, priors); and
    with `passes`, the runner kept full through azh_begin_positions (every
    slot with a positions pass in flight: stone bytes and superko hashes up,
    logits, priors, legal actions and values back, through pinned
    staging)."""
    import numpy as np
    import workload as W
    n, H = w.cfg[0], w.cfg[1]
    st, tm = W.stones(w, B)
    hist = np.zeros((B, H, n * n), np.uint8)
    hist[:, 0] = st
    plies = np.ones(B, np.int32)
    sym = (np.arange(B) % 8).astype(np.uint8)
    g = np.random.default_rng(1)
    seen = [g.integers(0, 2 ** 63, seen_per_position, dtype=np.int64).astype(np.uint64) for _ in range(B)]
    enc, leg, pri, chain = (x / iters for x in r.time_positions(hist, tm, plies, sym, seen, iters))
    A, P = n * n, 2 * H + 2
    enc_bytes = B * (H * A + P * A * 4)                      # stone bytes in, planes out
    leg_bytes = B * (A + (A + 1) + 8 * seen_per_position)    # boards and superko hashes in, masks out
    kept = {}
    if passes:
        r.time_pipelined_positions(B, 4, hist, tm, plies, sym, seen)   # every slot's graph captured
        ms = r.time_pipelined_positions(B, passes, hist, tm, plies, sym, seen)
        kept = {"kept_full_positions_per_s": round(B * passes / (ms * 1e-3), 1),
                "kept_full_passes": passes,
                "host_bytes_in_per_position": H * A + 4 + 1 + 1 + 8 + 8 * seen_per_position,
                "planes_bytes_per_position": P * A * 4}
    return {
        "workload": f"{n}x{n} batch {B}, the benchmark's boards, {seen_per_position} superko hashes each",
        "encode_us": round(enc * 1e3, 2),
        "legal_us": round(leg * 1e3, 2),
        "priors_us": round(pri * 1e3, 2),
        "chain_ms": round(chain, 4),
        "chain_positions_per_s": round(B / (chain * 1e-3), 1),
        "encode_gbs": round(enc_bytes / (enc * 1e-3) / 1e9, 1),
        "legal_positions_per_s": round(B / (leg * 1e-3), 1),
        "legal_gbs": round(leg_bytes / (leg * 1e-3) / 1e9, 2),
        **kept,
        "_inputs": (st, tm, seen),
    }


def positions_cpu_baseline(w, st, tm, seen, H, budget_s=3.0):
    """The oracle's encodePlanes + legal moves (Board::isLegal, hashAfter,
    the superko scan) for the same positions on the host: one
    single-threaded worker per host CPU, as the pass's CPU baseline, each
    taking the positions in turn for budget_s seconds."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    workers, host = cpu_workers()
    rate, el = O.time_positions_workers(st, tm, w.cfg[0], H, seen, workers, budget_s)
    return {"value": round(rate, 1), "unit": "positions/s", "cores": workers, "host_cpus": host, "kind": "port",
            "sample": f"{workers} single-threaded workers (one per host CPU), {round(rate * el)} positions in "
                      f"{el:.1f} s (oracle encodePlanes + legal moves with superko)"}


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py: runs on one GPU only (asked for {args.gpus}); inference of independent "
              f"positions shards with no exchange step, one runner per GPU", file=sys.stderr)
        sys.exit(2)

    import azgo_hip
    import workload as W

    ok, why = azgo_hip.available()
    if not ok:
        raise SystemExit(f"bench.py: no usable gfx950 GPU: {why}")
    if args.mode == "copy-calibration":
        return copy_calibration(args.mib, args.conv_iters)
    if args.mode == "mfma-calibration":
        return mfma_calibration(args.conv_iters)
    if args.mode == "stem-heads":
        return stem_heads(args.workload, args.batch, args.conv_iters)
    w = W.WORKLOADS[args.workload]
    B = args.batch or w.batch
    n, H, blocks, F, V = w.cfg
    tensors = W.network_tensors(w.cfg)
    inp, _ = W.positions(w, B)
    cfg = azgo_hip.net_cfg(*w.cfg)

    with azgo_hip.Runner(cfg, tensors, B, 2) as r:
        r.input(0)[:B] = inp
        r.input(1)[:B] = inp
        r.stage(0, B)
        for _ in range(args.warmup):
            r.enqueue(0, B)
        r.synchronize(0)

        # The timed region: K passes, synchronized on both sides.
        r.synchronize(0)
        t0 = time.perf_counter()
        for _ in range(args.steps):
            r.enqueue(0, B)
        r.synchronize(0)
        dt = time.perf_counter() - t0
        ms_per_step = dt * 1e3 / args.steps
        value = B * args.steps / dt

        # The same passes timed with HIP events on the pass's stream, and the
        # median of single passes, each timed on its own.
        ev_ms = r.time_passes(0, B, args.steps) / args.steps
        ev_median_ms = statistics.median(r.time_passes(0, B, 1) for _ in range(args.steps))
        # The dominant kernel. A pass alone whose batch fills its rounds of
        # one workgroup per CU (the headline one) runs the stem and the tower
        # as one board-resident launch: timed as the pass launches it. Else
        # the tower's per-layer convolutions, one launch per layer over the
        # whole batch (timed either way, for the per-layer kernel's figure).
        # Each timing runs once untimed first: a kernel's first launch in the
        # process also loads it.
        resident = bool(r.pass_form(B) & r.FORM_RESIDENT)
        r.time_tower_convs(0, B, 1)
        tower_ms, launches, layers = r.time_tower_convs(0, B, args.conv_iters)
        layer_launch_ms = tower_ms / launches
        if resident:
            r.time_resident_tower(0, B, 1, stem=True)
            conv_ms = r.time_resident_tower(0, B, args.conv_iters, stem=True) / args.conv_iters
        # The tower as the pass runs it (board-resident, or two half-batch
        # chains on two streams where the pass splits): the effective time
        # per layer of the batch.
        r.time_tower_layers(0, B, 1)
        pass_tower_ms, pass_layers = r.time_tower_layers(0, B, args.conv_iters)
        layer_ms = pass_tower_ms / pass_layers
        # The matrix units' measured ceiling: dependent MFMA chains, one
        # 8-wave workgroup per CU, nothing else in the way.
        ceil_ms, ceil_flops = azgo_hip.probe_mfma(20000, 3)
        mfma_ceiling = ceil_flops / (ceil_ms / 3 * 1e-3) / 1e12
        # PCIe-inclusive round trips (pinned H2D, pass, D2H, wait), for the record.
        rt_ms = r.time_round_trips(0, B, max(3, args.steps // 5)) / max(3, args.steps // 5)
        rt_median_ms = statistics.median(r.time_round_trips(0, B, 1) for _ in range(max(3, args.steps // 5)))
        # The first pass at a batch size the slot has not run (its graph is
        # captured and instantiated then), against the same size once cached.
        capture = None
        if B > 1:
            new_b = B - 1
            first_ms = r.time_round_trips(0, new_b, 1)
            cached_ms = statistics.median(r.time_round_trips(0, new_b, 1) for _ in range(3))
            capture = {"batch": new_b, "first_round_trip_ms": round(first_ms, 4),
                       "cached_round_trip_ms": round(cached_ms, 4),
                       "capture_ms": round(first_ms - cached_ms, 4)}
        # Both slots kept full through begin/done, each pass with its own
        # pinned copies (the reference bench's "2-slot" GPU rate).
        two_slot = None
        if not args.no_two_slot:
            r.time_pipelined(B, 4)   # the second slot's graph is captured on its first pass
            pipe_passes = max(8, args.steps)
            two_slot = round(B * pipe_passes / (r.time_pipelined(B, pipe_passes) * 1e-3), 1)
        logits, values = r.fetch(0, B)
        assert (logits == logits).all() and (values == values).all(), "NaN in outputs"
        pos = None if args.no_positions else positions_leg(
            r, w, B, args.seen, passes=None if args.no_two_slot else max(8, args.steps))

    layer_launch_flops = w.trunk_conv_flops(B) * (layers // launches)
    if resident:
        conv_flops = w.stem_conv_flops(B) + w.trunk_conv_flops(B) * 2 * blocks
        kernel_name = (f"convTowerResident (the stem and the residual tower, each board resident in one workgroup: "
                       f"one launch = the pass's {1 + 2 * blocks} convolutions over the batch)")
    else:
        conv_ms = layer_launch_ms
        conv_flops = layer_launch_flops
        kernel_name = "conv3x3Tower (residual tower, one launch = one layer over the batch)"
    achieved = conv_flops / (conv_ms * 1e-3) / 1e12
    pass_tflops = w.flops_per_position() * B / (ms_per_step * 1e-3) / 1e12
    # "..., kernels <all> (conv <conv>)": the traffic profile is keyed by the convolution's own hash.
    kernel_hash = azgo_hip.describe().rsplit("(conv ", 1)[-1].rstrip(")")
    name = f"{n}x{n} {blocks}x{F} batch {B}"
    traffic = traffic_from_profile(name, kernel_hash, kernel_name.split(" ")[0])

    line = {
        "metric": "net evals (positions)/sec at 19x19 batch 256; % fp32-MFMA peak",
        "value": round(value, 1),
        "unit": "positions/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        # The reference's figure includes the pinned copies (both slots kept
        # full, apps/bench.cpp:227-279): compared with this build's rate
        # measured the same way, not with the device-resident `value`.
        "vs_baseline": (round(two_slot / REFERENCE_POS_PER_S, 3)
                        if args.workload == 3 and B == 256 and two_slot else None),
        "dtype": "fp32",
        "data": "synthetic (seeded He-normal weights, synthetic BN statistics, random boards)",
        "config": {"workload": name, "board": n, "blocks": blocks, "filters": F, "value_hidden": V,
                   "global_batch": B, "parallelism": "single GPU"},
        "pct_fp32_mfma_peak": round(100 * pass_tflops / PEAK_FP32_MFMA_TFLOPS, 2),
        "pass_tflops": round(pass_tflops, 2),
        "event_ms_per_step": round(ev_ms, 4),
        "event_median_ms_per_pass": round(ev_median_ms, 4),
        "round_trip_ms": round(rt_ms, 4),
        "round_trip_median_ms": round(rt_median_ms, 4),
        "two_slot_positions_per_s": two_slot,
        "new_batch_size": capture,
        "roofline": {
            "kernel": kernel_name,
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_FP32_MFMA_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_FP32_MFMA_TFLOPS, 4),
            "traffic": traffic,
            # HBM bandwidth of one launch from the counters: traffic / launch time.
            "traffic_gb_s": round(traffic / (conv_ms * 1e-3) / 1e9, 1) if traffic else None,
            "avg_launch_ms": round(conv_ms, 4),
            "per_layer_ms": round(layer_ms, 4),
            "per_layer_frac": round(w.trunk_conv_flops(B) / (layer_ms * 1e-3) / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4),
            "flops_per_launch": conv_flops,
            # The published peak assumes 2.4 GHz; under a full MFMA load the
            # chip runs slower. Beside `frac`: the same kernel against the
            # rate measured for MFMAs alone in this run.
            "measured_mfma_ceiling": round(mfma_ceiling, 2),
            "frac_of_measured_ceiling": round(achieved / mfma_ceiling, 4),
            # The per-layer convolution kernel over the whole batch (the
            # dominant kernel where the pass launches per layer).
            "layer_launch": {
                "kernel": "conv3x3Tower",
                "avg_launch_ms": round(layer_launch_ms, 4),
                "frac": round(layer_launch_flops / (layer_launch_ms * 1e-3) / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4),
            },
        },
        "device": azgo_hip.describe(),
    }
    if not args.no_cpu:
        cb = cpu_baseline(args.workload, args.cpu_calls)
        line["cpu_baseline"] = cb
        line["gpu_over_cpu"] = round(value / cb["value"], 1) if cb["value"] > 0 else None
    else:
        line["cpu_baseline"] = None
    if pos is not None:
        st, tm, seen = pos.pop("_inputs")
        if not args.no_cpu:
            pos["cpu_baseline"] = positions_cpu_baseline(w, st, tm, seen, H)
        line["positions"] = pos
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
