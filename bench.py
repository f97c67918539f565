"""Benchmark of the RWKV-7 WKV-7 decode step on one MI355X.

Workload (one step): 128 active sequences, T=1, H=32 heads of 64, fp32 state
held in a 512-slot pool [512,32,64,64]; the kernel gathers each sequence's
state from pool[slot], applies one WKV-7 token, and scatters it back in place
(vkwr_v1_wkv::wkv_forward_slots_fp32).  Every step reads fresh r/w/k/v/a/b,
all generated (seeded, synthetic) and resident in HBM before timing.

The K timed steps are captured into one HIP graph (one kernel node per step,
each pointing at its own inputs) and replayed once, so the measurement is the
device's throughput, not Python's launch rate.  HIP events on the launch stream
bracket the replay; value = algorithmic bytes per step / time per step.

Prints one JSON line (rank 0).  `--gpus N` with N > 1 is refused: this build
measures one GPU.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import torch  # noqa: E402  (before vkwr_amd: shared HIP runtime)

P_SLOTS, B_ACTIVE, H, HEAD = 512, 128, 32, 64
C = H * HEAD
HBM_PEAK_GBS = 8000.0
# Algorithmic bytes per step: fp32 state read + write, 6 fp16 inputs, fp16 y, int32 slots.
STATE_BYTES = B_ACTIVE * H * HEAD * HEAD * 4
STEP_BYTES = 2 * STATE_BYTES + 6 * B_ACTIVE * C * 2 + B_ACTIVE * C * 2 + B_ACTIVE * 4
PROFILE_SUMMARY = os.path.join(ROOT, "profiles", "wkv7_fp32_slots_decode_c1.md")


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="target length of the CPU baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    return ap.parse_args()


def make_inputs(n_steps, device, seed=0, chunk=64):
    """[n_steps, 6, B, 1, C] fp16 following BASELINE config 0's distributions."""
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.empty(n_steps, 6, B_ACTIVE, 1, C, dtype=torch.float16, device=device)
    for s0 in range(0, n_steps, chunk):
        n = min(chunk, n_steps - s0)
        shp = (n, B_ACTIVE, 1, C)
        r, k, v = (torch.randn(shp, device=device, generator=g) for _ in range(3))
        w = torch.exp(-0.6065 * torch.sigmoid(torch.randn(shp, device=device, generator=g)))
        kk = torch.nn.functional.normalize(k.half().float().view(n, B_ACTIVE, 1, H, HEAD), dim=-1)
        a_vec = torch.sigmoid(torch.randn(n, B_ACTIVE, 1, H, HEAD, device=device, generator=g))
        x[s0:s0 + n, 0] = r.half()
        x[s0:s0 + n, 1] = w.half()
        x[s0:s0 + n, 2] = k.half()
        x[s0:s0 + n, 3] = v.half()
        x[s0:s0 + n, 4] = (-kk).reshape(shp).half()
        x[s0:s0 + n, 5] = (kk * a_vec).reshape(shp).half()
    return x


def read_traffic():
    """HBM bytes per launch measured with rocprofv3 counters (profiles/ summary), or None."""
    try:
        for line in open(PROFILE_SUMMARY):
            if line.strip().startswith("traffic_bytes_per_launch:"):
                return float(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


def capture(step_fn, n_steps, stream):
    """Capture n_steps calls of step_fn(i) into one HIP graph."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(g, stream=stream):
            for i in range(n_steps):
                step_fn(i)
    torch.cuda.synchronize()
    return g


def cpu_baseline(target_s):
    """Oracle (C restatement, OpenMP over heads) on the host cores, bounded sample."""
    import numpy as np

    from oracle import oracle as orc
    from tests.wkv_inputs import make_state, make_wkv_inputs

    cores = len(os.sched_getaffinity(0))
    orc.set_threads(cores)
    pool = make_state(P_SLOTS, H, seed=0)
    slots = np.random.default_rng(0).permutation(P_SLOTS)[:B_ACTIVE]
    sets = [make_wkv_inputs(B_ACTIVE, 1, H, seed=s) for s in range(4)]
    orc.wkv_fp32_slots(B_ACTIVE, 1, C, H, pool, slots, *sets[0])  # warm-up
    n, t0 = 0, time.perf_counter()
    while True:
        orc.wkv_fp32_slots(B_ACTIVE, 1, C, H, pool, slots, *sets[n % 4])
        n += 1
        dt = time.perf_counter() - t0
        if dt >= target_s or n >= 100000:
            break
    return {
        "value": round(STEP_BYTES * n / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{n} decode steps of config 1 (128 seqs x 32 heads, T=1, gather/step/scatter "
                  f"on a 512-slot pool) in {dt:.1f} s; {dt / n * 1e3:.2f} ms/step, "
                  f"{B_ACTIVE * n / dt:.0f} tokens/s",
    }


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the WKV path shards by sequence with no communication; see DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    assert torch.cuda.is_available(), "no GPU visible"
    import vkwr_amd  # noqa: F401
    from vkwr_amd._ops.v1 import v1_wkv_ops as ops

    dev = torch.device("cuda:0")
    K, W = args.steps, args.warmup
    gen = torch.Generator().manual_seed(0)
    pool = (torch.randn(P_SLOTS, H, HEAD, HEAD, generator=gen) * 0.1).to(dev)
    perm = torch.randperm(P_SLOTS, generator=gen)
    slots = perm[:B_ACTIVE].to(torch.int32).to(dev)
    ops.validate_slots(slots, P_SLOTS)
    inputs = make_inputs(K + W, dev)  # fresh inputs for every step, ~3.3 GB at K=1000
    y = torch.empty(B_ACTIVE, 1, C, dtype=torch.float16, device=dev)
    op = torch.ops.vkwr_v1_wkv.wkv_forward_slots_fp32

    def step(i, sl=slots):
        x = inputs[i]
        op(B_ACTIVE, 1, C, H, pool, sl, x[0], x[1], x[2], x[3], x[4], x[5], y)

    for i in range(W):
        step(K + i)
    torch.cuda.synchronize()

    stream = torch.cuda.Stream()
    graph = capture(step, K, stream)
    graph.replay()  # one untimed replay (first replay uploads the graph)
    torch.cuda.synchronize()

    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        ev0.record(stream)
        graph.replay()
        ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = ev0.elapsed_time(ev1)
    ms_per_step = gpu_ms / K
    gbs = STEP_BYTES / (ms_per_step * 1e-3) / 1e9

    # Cold(er)-cache variant: rotate 4 disjoint 128-slot sets (the whole 256 MiB pool).
    sets = [perm[i * B_ACTIVE:(i + 1) * B_ACTIVE].to(torch.int32).to(dev) for i in range(4)]
    kc = min(K, 400)
    graph_c = capture(lambda i: step(i, sets[i % 4]), kc, stream)
    graph_c.replay()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        ev0.record(stream)
        graph_c.replay()
        ev1.record(stream)
    torch.cuda.synchronize()
    cold_ms = ev0.elapsed_time(ev1) / kc
    del graph, graph_c

    traffic = read_traffic()
    result = {
        "metric": "WKV-7 decode HBM GB/s (% peak); decode tokens/s at 1.5B-shape bs=128",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded; BASELINE config 0/1 distributions, resident in HBM)",
        "config": {"workload": "wkv7_decode_slot_pool (BASELINE config 1)", "pool_slots": P_SLOTS,
                   "active_seqs": B_ACTIVE, "heads": H, "head_size": HEAD, "T": 1,
                   "state": "fp32", "io": "fp16", "timing": "HIP graph of K steps, HIP events"},
        "tokens_per_s": round(B_ACTIVE / (ms_per_step * 1e-3), 1),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "bytes_per_launch": STEP_BYTES},
        "variants": {
            "rotating_4_slot_sets": {"ms_per_step": round(cold_ms, 5),
                                     "GB/s": round(STEP_BYTES / (cold_ms * 1e-3) / 1e9, 2),
                                     "note": "4 disjoint 128-slot sets cycled: 256 MiB working set"},
            "wall_s_timed_region": round(wall, 4),
        },
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
