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
import traceback
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import torch  # noqa: E402  (before vkwr: shared HIP runtime)

P_SLOTS, B_ACTIVE, H, HEAD = 512, 128, 32, 64
C = H * HEAD
HBM_PEAK_GBS = 8000.0
# Algorithmic bytes per step: fp32 state read + write, 6 fp16 inputs, fp16 y, int32 slots.
STATE_BYTES = B_ACTIVE * H * HEAD * HEAD * 4
STEP_BYTES = 2 * STATE_BYTES + 6 * B_ACTIVE * C * 2 + B_ACTIVE * C * 2 + B_ACTIVE * 4
COLD_SLOTS = 2048  # cold-cache variant: 1 GiB pool
PROFILE_SUMMARY = os.path.join(ROOT, "profiles", "wkv7_fp32_step_kernel_decode_c1.md")


_T0 = time.perf_counter()


def log(msg):
    """Progress on stderr (stdout carries only the JSON line)."""
    print(f"bench [{time.perf_counter() - _T0:6.1f} s] {msg}", file=sys.stderr, flush=True)


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="target length of the CPU baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--model-steps", type=int, default=20,
                    help="timed decode steps of the 1.5B-shape model at bs=128 (0: skip)")
    ap.add_argument("--prefill-calls", type=int, default=20,
                    help="timed calls of the config-2 prefill (B=8, T=1024, H=32; 0: skip)")
    ap.add_argument("--serve-steps", type=int, default=3,
                    help="timed steps of the 7B mixed prefill+decode step (BASELINE config 4; 0: skip)")
    ap.add_argument("--sampling-calls", type=int, default=50,
                    help="timed calls per sampling setting at bs=128 over the 65536-token vocabulary (0: skip)")
    ap.add_argument("--rowmajor-gemm", action="store_true",
                    help="run the model decode step on the row-major GEMM instead of the frag GEMM")
    ap.add_argument("--eager", action="store_true",
                    help="launch every step directly instead of replaying a HIP graph (for counter runs); "
                         "skips the cache variants")
    ap.add_argument("--ops-calls", type=int, default=30,
                    help="timed calls per shape of the op-surface GEMMs at M=1 and M=128 (0: skip)")
    ap.add_argument("--fp16-steps", type=int, default=200,
                    help="steps of the fp16-state WKV decode op at the config-1 shape (0: skip the fp16 section)")
    ap.add_argument("--only", choices=["decode", "prefill", "serve", "sampling", "ops", "fp16", "c1", "gemm7b"],
                    help="run one section alone and print its JSON object (for profiler runs); with --eager "
                         "the decode steps are launched directly")
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


def copy_calibration(dev, n_bytes=256 << 20, reps=3):
    """A plain device copy of known size (torch's copy kernel), run before the timed
    region so that a counter run (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE) sees a
    reference dispatch that moves exactly n_bytes each way."""
    src = torch.empty(n_bytes // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def capture(step_fn, n_steps, stream):
    """Capture n_steps calls of step_fn(i) into one HIP graph."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(g, stream=stream):
            for i in range(n_steps):
                step_fn(i)
    torch.cuda.synchronize()
    return g


def op_surface_decode(model, dev, steps, warmup=3):
    """The same config-3 decode step composed only of the reference's op surface
    (vkwr.model_executor.OpDecodeEngine: vkwr._ops wrappers, the batch's token-shift rows
    of every layer gathered with index_select at the start of the step and written back
    with index_copy_ at its end, WKV through the slot-pool op)
    on a row-major 160-slot pool: device time of one step captured into a HIP graph and
    replayed, and the eager step (host dispatch of ~400 op calls included)."""
    from vkwr_amd import capi
    from vkwr.model_executor import OpDecodeEngine, RWKV7State

    cfg, B = model.cfg, 128
    state = RWKV7State(cfg, 160, dev, std=0.1, seed=1, layout=capi.WKV_STATE_STD)
    eng = OpDecodeEngine(model)
    g = torch.Generator().manual_seed(3)
    slots = torch.randperm(160, generator=g)[:B].to(torch.int32).to(dev)
    tokens = torch.randint(0, cfg.vocab, (B,), generator=g, dtype=torch.int32).to(dev)
    for _ in range(warmup):
        eng.step(state, tokens, slots)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        ev0.record(stream)
        for _ in range(steps):
            eng.step(state, tokens, slots)
        ev1.record(stream)
    torch.cuda.synchronize()
    ms_eager = ev0.elapsed_time(ev1) / steps
    graph = capture(lambda i: eng.step(state, tokens, slots), 1, stream)
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        ev0.record(stream)
        for _ in range(steps):
            graph.replay()
        ev1.record(stream)
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / steps
    del graph, state, eng
    torch.cuda.empty_cache()
    return {"ms_per_step": round(ms, 4), "tokens_per_s": round(B / (ms * 1e-3), 1),
            "ms_per_step_eager": round(ms_eager, 4), "tokens_per_s_eager": round(B / (ms_eager * 1e-3), 1),
            "steps": steps,
            "path": "OpDecodeEngine: reference op wrappers only (add_layer_norm_tmix_mix6_f16, linear_f16_orig, relu_square, "
                    "linear_wag(v)_rank_in/out_f16, add_vec, tmix_kk_a_gate, wkv_forward_slots_fp32, "
                    "tmix_lnx_rkvres_xg, add_layer_norm_cmix_mix_f16, "
                    "add_last_layer_norm_f16), shift rows of all layers gathered / scattered once per step "
                    "with index_select / index_copy_",
            "timing": "ms_per_step: one step captured as a HIP graph and replayed (device time); "
                      "ms_per_step_eager: op calls issued from Python every step"}


def model_decode(dev, steps, warmup=3, frag=True, eager=False, keep_cpu_model=None, op_steps=0):
    """the RWKV-7 1.5B-shape decode step (L=24, C=2048, random fp16
    weights) for 128 sequences at T=1 from a 160-slot state pool.  One step is captured
    into a HIP graph and replayed `steps` times (the recurrent state advances every
    replay); HIP events on the replay stream time it.  eager=True launches every step
    directly (profiler counter runs)."""
    from vkwr.model_executor import DecodeEngine, RWKV7Config, RWKV7Model, RWKV7State
    from vkwr.model_executor.rwkv7 import flops_per_step, gbytes_per_step

    cfg = RWKV7Config.preset("1.5b")
    B = 128
    model = RWKV7Model(cfg, dev, seed=0)
    from vkwr_amd import capi
    state = RWKV7State(cfg, 160, dev, std=0.1, seed=1,
                       layout=capi.WKV_STATE_ILV if frag else capi.WKV_STATE_STD)
    eng = DecodeEngine(model, B, frag=frag)
    g = torch.Generator().manual_seed(3)
    slots = torch.randperm(160, generator=g)[:B].to(torch.int32).to(dev)
    tokens = torch.randint(0, cfg.vocab, (B,), generator=g, dtype=torch.int32).to(dev)
    for _ in range(warmup):
        eng.step(state, tokens, slots)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if eager:
        with torch.cuda.stream(stream):
            ev0.record(stream)
            for _ in range(steps):
                eng.step(state, tokens, slots)
            ev1.record(stream)
        torch.cuda.synchronize()
    else:
        graph = capture(lambda i: eng.step(state, tokens, slots), 1, stream)
        for _ in range(warmup):
            graph.replay()
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            ev0.record(stream)
            for _ in range(steps):
                graph.replay()
            ev1.record(stream)
        torch.cuda.synchronize()
        del graph
    ms = ev0.elapsed_time(ev1) / steps
    del eng, state
    torch.cuda.empty_cache()
    op = op_surface_decode(model, dev, op_steps) if op_steps > 0 else None
    if keep_cpu_model is not None:
        keep_cpu_model.append(cpu_model_copy(model))
    nbytes = gbytes_per_step(cfg, B)
    gbs = nbytes / (ms * 1e-3) / 1e9
    out = {
        "workload": "RWKV-7 1.5B-shape decode step (BASELINE config 3): L=24, C=2048, H=32, F=8192, "
                    "ranks w/a/v/g 96/96/64/256, V=65536, bs=128, T=1, random-init fp16 weights, "
                    "fp32 WKV state in a 160-slot pool",
        "tokens_per_s": round(B / (ms * 1e-3), 1),
        "ms_per_step": round(ms, 4),
        "steps": steps,
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_step": nbytes,
                     "tokens_per_s_at_peak": round(B / (nbytes / (HBM_PEAK_GBS * 1e9)), 1)},
        "gemm_tflops": round(flops_per_step(cfg, B) / (ms * 1e-3) / 1e12, 2),
        "gemm_path": "frag (vkwr_frag_gemm_f16, weights packed at load)" if frag else "row-major (vkwr_gemm_f16)",
        "timing": ("eager launches" if eager else "one decode step captured as a HIP graph, replayed") +
                  "; HIP events on the launch stream",
    }
    if op is not None:
        out["op_surface_step"] = op
    return out


def prefill_c2(dev, steps, warmup=100):
    """WKV-7 prefill, B=8 sequences x T=1024 tokens, H=32, fp32 state
    gathered from / scattered back to random slots of the 512-slot pool in the same call
    (vkwr_v1_wkv::wkv_forward_slots_fp32 -> the chunked prefill kernel).  Inputs drawn as
    in config 0, resident in HBM; eager calls (each is hundreds of microseconds) bracketed
    by HIP events on the current stream.  100 untimed calls first (~17 ms): the chip's clock
    ramps over the first ~150 calls from idle (the first 20 took ~12 % longer each than the
    steady state), which a short warm-up left inside the timed calls."""
    from vkwr._ops.v1 import v1_wkv_ops as ops

    Bp, Tp = 8, 1024
    g = torch.Generator(device=dev).manual_seed(2)
    shp = (Bp, Tp, C)
    r, k, v = (torch.randn(shp, device=dev, generator=g).half() for _ in range(3))
    w = torch.exp(-0.6065 * torch.sigmoid(torch.randn(shp, device=dev, generator=g))).half()
    kk = torch.nn.functional.normalize(k.float().view(Bp, Tp, H, HEAD), dim=-1)
    a_vec = torch.sigmoid(torch.randn(Bp, Tp, H, HEAD, device=dev, generator=g))
    a = (-kk).reshape(shp).half()
    b = (kk * a_vec).reshape(shp).half()
    pool = (torch.randn(P_SLOTS, H, HEAD, HEAD, device=dev, generator=g) * 0.1)
    slots = torch.randperm(P_SLOTS, device=dev, generator=g)[:Bp].to(torch.int32)
    y = torch.empty(shp, dtype=torch.float16, device=dev)
    call = lambda: torch.ops.vkwr_v1_wkv.wkv_forward_slots_fp32(Bp, Tp, C, H, pool, slots, r, w, k, v, a, b, y)
    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(steps):
        call()
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / steps
    nbytes = 7 * Bp * Tp * C * 2 + 2 * Bp * H * HEAD * HEAD * 4 + Bp * 4
    gbs = nbytes / (ms * 1e-3) / 1e9
    # algorithmic flops of the recurrence: per token, head and state element 9 -- the decay
    # multiply, the two multiply-adds of the update (s*d + sa*b + k*v) and one multiply-add
    # in each of the two dot products (sa = S a, y = S' r)
    alg_flops = Bp * Tp * H * HEAD * HEAD * 9
    # matrix-core work the chunked kernel actually issues per 16-token chunk and head: 4 state
    # waves x 80 v_mfma_f32_16x16x4_f32 (2048 flops each), 4 x 16 for the chunk matrices, 36 for
    # W^T (includes the W^T power series and padded tokens, so it is not a roofline numerator)
    mfma_flops = Bp * H * ((Tp + 15) // 16) * (4 * 80 + 4 * 16 + 36) * 2048
    # the reference-order (bit-exact) form of the same prefill: wkv_forward_seq_fp32 on a
    # dense state (one chain per dot product, token by token)
    st = pool[slots.long()].clone()
    seq = lambda: ops.wkv_forward_seq_fp32(Bp, Tp, C, H, st, r, w, k, v, a, b)  # noqa: E731
    for _ in range(5):
        seq()
    torch.cuda.synchronize()
    seq_calls = 10
    ev0.record()
    for _ in range(seq_calls):
        seq()
    ev1.record()
    torch.cuda.synchronize()
    ms_seq = ev0.elapsed_time(ev1) / seq_calls
    del r, w, k, v, a, b, pool, y, st
    torch.cuda.empty_cache()
    tflops = alg_flops / (ms * 1e-3) / 1e12
    return {
        "workload": "WKV-7 prefill (BASELINE config 2): B=8, T=1024, H=32, fp32 state in a 512-slot pool "
                    "(gather + scatter in the call), fp16 inputs drawn as in config 0",
        "tokens_per_s": round(Bp * Tp / (ms * 1e-3), 1),
        "hbm_GBps": round(gbs, 2),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "bytes_per_call": nbytes,
        "ms_per_call": round(ms, 4),
        "calls": steps,
        "ns_per_token_step": round(ms * 1e6 / Tp, 1),
        "roofline": {"bound": "mfma (fp32 matrix cores: 16-token chunks, one dependent chain of chunk "
                              "products per head)",
                     "achieved": round(tflops, 2), "peak": 157.3, "unit": "TFLOP/s",
                     "frac": round(tflops / 157.3, 4), "flops_per_call": alg_flops,
                     "flops": "algorithmic: 9 per token, head and state element",
                     "hbm_GBps": round(gbs, 2), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_call": nbytes},
        "issued_mfma_util": {"issued_flops_per_call": mfma_flops,
                             "TFLOP/s": round(mfma_flops / (ms * 1e-3) / 1e12, 2),
                             "frac_of_fp32_matrix_peak": round(mfma_flops / (ms * 1e-3) / 1e12 / 157.3, 4),
                             "note": "how busy the chunked form keeps the matrix cores (its own products, "
                                     "padded tokens and the W^T power series included); not a roofline"},
        "kernel": "wkv7_fp32_chunk_kernel (one 512-lane workgroup per (sequence, head): 4 state waves + 4 "
                  "waves preparing later chunks; 16-token chunks on v_mfma_f32_16x16x4_f32)",
        "reference_order_seq_fp32": {
            "ms_per_call": round(ms_seq, 4), "tokens_per_s": round(Bp * Tp / (ms_seq * 1e-3), 1),
            "ns_per_token_step": round(ms_seq * 1e6 / Tp, 1), "calls": seq_calls,
            "what": "wkv_forward_seq_fp32 on a dense [8,32,64,64] state, same inputs: the bit-exact "
                    "reference-order path (wkv7_fp32_seq_lat_kernel, one wave per (sequence, head))"},
    }


def wkv_fp16_family(dev, steps, seq_calls=20, warmup=5):
    """The fp16-state WKV ops (vkwr_v1_wkv::wkv_one_fp16 / wkv_seq_fp16, fp16 state [B,H,64,64],
    8 KiB per head; reference csrc/v1/wkv/wkv_fp16_v2.cu).  (1) wkv_one_fp16 at the config-1
    shape: 128 sequences x 32 heads, T=1, fresh r/w/k/v/a/b per step (config-0
    distributions), `steps` steps captured into one HIP graph and replayed; also over 32
    state tables cycled (1 GiB: the state comes from HBM, not the Infinity Cache).
    (2) wkv_seq_fp16 at the config-2 shape (B=8, T=1024, H=32), eager calls after 100
    untimed ones.  HIP events on the launch stream."""
    Bd = B_ACTIVE
    n = steps + warmup
    inputs = make_inputs(n, dev, seed=9)
    g = torch.Generator(device=dev).manual_seed(9)
    state = (torch.randn(Bd, H, HEAD, HEAD, device=dev, generator=g) * 0.1).half()
    y = torch.empty(Bd, C, dtype=torch.float16, device=dev)
    el = torch.zeros(Bd, dtype=torch.int32, device=dev)
    op = torch.ops.vkwr_v1_wkv.wkv_one_fp16

    def step(i, st=state):
        x = inputs[i]
        op(Bd, C, H, st, x[0].view(Bd, C), x[1].view(Bd, C), x[2].view(Bd, C), x[3].view(Bd, C),
           x[4].view(Bd, C), x[5].view(Bd, C), y, el)

    for i in range(warmup):
        step(steps + i)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed_graph(fn, k):
        gr = capture(fn, k, stream)
        gr.replay()
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            ev0.record(stream)
            gr.replay()
            ev1.record(stream)
        torch.cuda.synchronize()
        del gr
        return ev0.elapsed_time(ev1) / k

    ms_hot = timed_graph(step, steps)
    tables = torch.empty(32, Bd, H, HEAD, HEAD, dtype=torch.float16, device=dev).normal_(0.0, 0.1)
    ms_cold = timed_graph(lambda i: step(i, tables[i % 32]), steps)
    del tables, inputs
    one_bytes = 2 * Bd * H * HEAD * HEAD * 2 + 7 * Bd * C * 2 + Bd * 4
    out = {"wkv_one_fp16_c1_shape": {
        "ms_per_step": round(ms_hot, 5), "tokens_per_s": round(Bd / (ms_hot * 1e-3), 1),
        "GB/s": round(one_bytes / (ms_hot * 1e-3) / 1e9, 2),
        "hbm_frac": round(one_bytes / (ms_hot * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "bytes_per_step": one_bytes,
        "cold_32_tables": {"ms_per_step": round(ms_cold, 5),
                           "GB/s": round(one_bytes / (ms_cold * 1e-3) / 1e9, 2),
                           "hbm_frac": round(one_bytes / (ms_cold * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
        "workload": "128 sequences x 32 heads, T=1, fp16 state 32 MiB (read + written), fresh fp16 inputs "
                    "per step; cold: 32 state tables (1 GiB) cycled"}}
    # (2) prefill at the config-2 shape
    Bp, Tp = 8, 1024
    shp = (Bp, Tp, C)
    r, k, v = (torch.randn(shp, device=dev, generator=g).half() for _ in range(3))
    w = torch.exp(-0.6065 * torch.sigmoid(torch.randn(shp, device=dev, generator=g))).half()
    kk = torch.nn.functional.normalize(k.float().view(Bp, Tp, H, HEAD), dim=-1)
    a = (-kk).reshape(shp).half()
    b = (kk * torch.sigmoid(torch.randn(Bp, Tp, H, HEAD, device=dev, generator=g))).reshape(shp).half()
    st = (torch.randn(Bp, H, HEAD, HEAD, device=dev, generator=g) * 0.1).half()
    yp = torch.empty(shp, dtype=torch.float16, device=dev)
    elp = torch.zeros(Bp, dtype=torch.int32, device=dev)
    call = lambda: torch.ops.vkwr_v1_wkv.wkv_seq_fp16(Bp, Tp, C, H, st, r, w, k, v, a, b, yp, elp)  # noqa: E731
    for _ in range(100):
        call()
    torch.cuda.synchronize()
    ev0.record()
    for _ in range(seq_calls):
        call()
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / seq_calls
    seq_bytes = 7 * Bp * Tp * C * 2 + 2 * Bp * H * HEAD * HEAD * 2 + Bp * 4
    flops = Bp * Tp * H * HEAD * HEAD * 9
    out["wkv_seq_fp16_c2_shape"] = {
        "ms_per_call": round(ms, 4), "tokens_per_s": round(Bp * Tp / (ms * 1e-3), 1),
        "ns_per_token_step": round(ms * 1e6 / Tp, 1),
        "GB/s": round(seq_bytes / (ms * 1e-3) / 1e9, 2),
        "hbm_frac": round(seq_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "fp16_TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 2),
        "calls": seq_calls,
        "workload": "B=8, T=1024, H=32, fp16 state, inputs drawn as in config 0; 256 (sequence, head) "
                    "chains of 1024 dependent tokens (latency-bound: 256 waves on 1024 SIMDs)",
        "kernel": "wkv7_fp16_seq_kernel<false>: T > 1 with at most 4 x CUs chains"}
    del r, w, k, v, a, b, st, yp
    torch.cuda.empty_cache()
    out["kernel"] = ("wkv7_fp16_kernel<false> (T = 1) and wkv7_fp16_seq_kernel<false> (T > 1, few chains), "
                     "vkwr_amd/csrc/wkv.hip: one wave64 per (sequence, head)")
    out["timing"] = "decode: HIP graph of the steps, HIP events on the replay stream; prefill: eager calls"
    return out


def sampling_bs128(dev, calls, warmup=3):
    """Token sampling after the config-3 decode step: 128 rows of fp32 logits over the
    65536-token vocabulary, resident in HBM (vkwr_sampling ops, one 1024-lane workgroup
    per row).  Eager calls bracketed by HIP events on the current stream."""
    from vkwr._ops import sampling_ops as ops

    Bs, Vs = 128, 65536
    g = torch.Generator(device=dev).manual_seed(5)
    logits = torch.randn(Bs, Vs, device=dev, generator=g) * 3.0
    pens = torch.zeros(Bs, Vs, device=dev)
    states = ops.setup_rand(1234, Bs)
    settings = {
        "untruncated": lambda: ops.temperature_topk_topp(logits, states, 1.0, -1, 1.0),
        "greedy": lambda: ops.temperature_topk_topp(logits, states, 1.0, 1, 1.0),
        "top_k40_top_p0.9": lambda: ops.temperature_topk_topp(logits, states, 0.8, 40, 0.9),
        "penalties_top_k40_top_p0.9": lambda: ops.repetition_topk_topp(logits, pens, states, 0.5, 0.5, 0.996, 0.8,
                                                                        40, 0.9),
    }
    out = {}
    for name, call in settings.items():
        for _ in range(warmup):
            call()
        torch.cuda.synchronize()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        for _ in range(calls):
            call()
        ev1.record()
        torch.cuda.synchronize()
        us = ev0.elapsed_time(ev1) * 1000 / calls
        nbytes = Bs * Vs * 4 * (4 if name.startswith("penalties") else 1)  # logits (+ penalties read twice, written)
        gbs = nbytes / (us * 1e-6) / 1e9
        out[name] = {"us_per_call": round(us, 2), "rows_per_s": round(Bs / (us * 1e-6), 1),
                     "hbm_gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
    del logits, pens, states
    torch.cuda.empty_cache()
    return {
        "workload": "token sampling, B=128 rows x V=65536 fp32 logits (the config-3 decode step's head output)",
        "calls": calls,
        "settings": out,
        "roofline_note": "VALU-bound: one 1024-lane workgroup per row keeps 64 logits per lane in registers and "
                         "makes ~15 vector operations per logit (128 rows fill half of the 256 CUs)",
        "kernel": "sampling_kernel<16> (vkwr_amd/csrc/sampling.hip)",
    }


def ops_small_m(dev, calls, warmup=3):
    """The reference op surface at decode sizes: vkwr_v1_linear ops (torch.ops, row-major
    weights as the reference's callers pass them) at M = 1 (the reference's GEMV table:
    head 2048 -> 65536, 4096 -> 4096, 4096 -> 16384, [K,N] weights of linear_f16) and at
    M = 128 (the 1.5B projection shapes, nn.Linear [N,K] weights of linear_f16_orig),
    beside the decode driver's frag-layout GEMM on the same M = 128 shapes.  Weights are
    rotated over copies spanning >= 512 MiB, so every call streams them from HBM."""
    from vkwr_amd import capi
    from vkwr._ops.v1 import v1_linear_ops as L

    g = torch.Generator(device=dev).manual_seed(11)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    stream = torch.cuda.Stream()

    def timed(fn, n):
        """Device time per call: n calls captured into one HIP graph, replayed once after an
        untimed replay (the op surface's host-side dispatch is not what is measured)."""
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        graph = capture(fn, n, stream)
        graph.replay()
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            ev0.record(stream)
            graph.replay()
            ev1.record(stream)
        torch.cuda.synchronize()
        del graph
        return ev0.elapsed_time(ev1) / n * 1e3  # us

    def copies(shape):
        nb = shape[0] * shape[1] * 2
        n = max(2, -(-(512 << 20) // nb))
        return [(torch.randn(*shape, device=dev, generator=g) * 0.02).half() for _ in range(n)]

    out = {}
    for (K, N) in ((2048, 65536), (4096, 4096), (4096, 16384)):
        ws = copies((K, N))
        x = torch.randn(1, K, device=dev, generator=g).half()
        us = timed(lambda i: L.linear_f16(x, ws[i % len(ws)]), calls)
        gbs = K * N * 2 / (us * 1e-6) / 1e9
        out[f"m1_linear_f16_K{K}_N{N}"] = {"us": round(us, 2), "weight_GBps": round(gbs, 1),
                                           "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
        del ws
    for (K, N) in ((2048, 65536), (4096, 4096)):  # nn.Linear [N,K] weights (linear_f16_orig)
        ws = copies((N, K))
        x = torch.randn(1, K, device=dev, generator=g).half()
        us = timed(lambda i: L.linear_f16_orig(x, ws[i % len(ws)]), calls)
        gbs = K * N * 2 / (us * 1e-6) / 1e9
        out[f"m1_linear_f16_orig_K{K}_N{N}"] = {"us": round(us, 2), "weight_GBps": round(gbs, 1),
                                                "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
        del ws
    # the activation-sparse FFN down projection at M = 1: relu^2 of a N(0,1) pre-activation
    # leaves about half of the F rows zero, and only the other rows of value_fc are read
    from vkwr._ops.v1 import v1_mix_ops as MX
    for (C, F) in ((2048, 8192), (4096, 16384)):
        ws = copies((F, C))
        pre = torch.randn(F, device=dev, generator=g).half()
        live = int((pre > 0).sum())
        us = timed(lambda i: MX.cmix_sparse_down_relu_one(C, F, pre, ws[i % len(ws)]), calls)
        dense_x = pre.view(1, F).abs() + 0.01  # no zero row
        us_dense = timed(lambda i: L.linear_f16(dense_x, ws[i % len(ws)]), calls)
        read = live * C * 2
        out[f"m1_cmix_sparse_down_relu_one_C{C}_F{F}"] = {
            "us": round(us, 2), "rows_read_frac": round(live / F, 4),
            "read_GBps": round(read / (us * 1e-6) / 1e9, 1),
            "hbm_frac": round(read / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "dense_weight_GBps": round(F * C * 2 / (us * 1e-6) / 1e9, 1),
            "dense_activation_us": round(us_dense, 2)}
        del ws
    for (K, N, role) in ((2048, 2048, "r/k/v/o"), (2048, 8192, "ffn_key"), (8192, 2048, "ffn_value")):
        ws = copies((N, K))
        x = torch.randn(128, K, device=dev, generator=g).half()
        us = timed(lambda i: L.linear_f16_orig(x, ws[i % len(ws)]), calls)
        # the decode driver's path: both operands packed in the frag layout
        xf = capi.frag_empty(128, K, dev)
        capi.frag_pack(x, 128, K, xf)
        wf = []
        for w in ws:
            f = capi.frag_empty(N, K, dev, zero=False)
            capi.frag_pack(w, N, K, f)
            wf.append(f)
        del ws
        y = torch.empty(128, N, dtype=torch.float16, device=dev)
        us_frag = timed(lambda i: capi.frag_gemm([capi.frag_problem(xf, wf[i % len(wf)], y, 128, N, K)]), calls)
        gbs = N * K * 2 / (us * 1e-6) / 1e9
        out[f"m128_linear_f16_orig_{role}_K{K}_N{N}"] = {
            "us": round(us, 2), "weight_GBps": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "frag_path_us": round(us_frag, 2), "vs_frag": round(us / us_frag, 3)}
        del wf
        torch.cuda.empty_cache()
    # the rest of the 1.5B layer's op-surface GEMMs at M = 128: the low-rank adapters (one op
    # each, 4 problems) and the [K,N] activation-sparse FFN down projection
    from vkwr._ops.v1 import v1_rank_ops as RK
    Mr, Cr, Fr, Rw, Ra, Rg, Rv = 128, 2048, 8192, 96, 96, 64, 256
    rn = lambda *sh, sd=1.0: (torch.randn(*sh, device=dev, generator=g) * sd).half()  # noqa: E731
    xs = [rn(Mr, Cr) for _ in range(4)]
    ins = [[rn(r, Cr, sd=0.02) for r in (Rw, Ra, Rg, Rv)] for _ in range(16)]  # 16 x 1.1 MiB
    us = timed(lambda i: RK.linear_wagv_rank_in_f16(Mr, Cr, Rw, Ra, Rg, Rv, *xs, *ins[i % 16]), calls)
    out["m128_linear_wagv_rank_in_f16"] = {"us": round(us, 2), "note": "4 problems, K=2048, N=96/96/64/256"}
    lows = [rn(Mr, r) for r in (Rw, Ra, Rg, Rv)]
    outs_w = [[rn(Cr, r, sd=0.1) for r in (Rw, Ra, Rg, Rv)] for _ in range(16)]
    v, vf, v0 = rn(Mr, Cr), rn(Mr, Cr), rn(Cr)
    us = timed(lambda i: RK.linear_wagv_rank_out_f16(Mr, Cr, Rw, Ra, Rg, Rv, *lows, *outs_w[i % 16], v, vf, v0), calls)
    out["m128_linear_wagv_rank_out_f16"] = {"us": round(us, 2),
                                            "note": "4 problems, N=2048, K=96/96/64/256, tanh / sigmoid on A, "
                                                    "value residual"}
    del ins, outs_w
    pre = rn(Mr, 1, Fr)
    vfc = copies((Fr, Cr))
    us = timed(lambda i: MX.cmix_sparse_down_relu_rows(Mr, 1, Cr, Fr, pre, vfc[i % len(vfc)]), calls)
    out["m128_cmix_sparse_down_relu_rows_C2048_F8192"] = {
        "us": round(us, 2), "note": "[K,N] value_fc: each workgroup streams 128-byte pieces of 4 KiB k rows"}
    del vfc
    torch.cuda.empty_cache()
    return {
        "workload": "vkwr_v1_linear ops through torch.ops at M=1 ([K,N] weights, linear_f16) and M=128 "
                    "([N,K] weights, linear_f16_orig), weights cold (rotated over >= 512 MiB of copies); "
                    "frag_path_us: the decode driver's frag GEMM on the same M=128 shapes (unpadded, one call); "
                    "m1_cmix_sparse_down_relu_one: vkwr_v1_mix's activation-sparse FFN down projection, "
                    "relu^2 of an N(0,1) pre-activation (read bytes = nonzero rows x C x 2; "
                    "dense_activation_us: the same GEMV with no zero row)",
        "calls": calls,
        "shapes": out,
        "timing": "each shape's calls captured into one HIP graph and replayed; HIP events on the replay "
                  "stream, mean per call",
    }


def serve_mixed_7b(dev, steps, warmup=1):
    """the RWKV-7 7B shape (L=32, C=4096, F=16384, random fp16 weights),
    one continuous-batching step = 256 decode rows + 4 prefill chunks of 512 tokens
    (2304 GEMM rows) on a 2048-slot fp32 state pool.  Eager launches (shapes vary per
    step in serving); HIP events on the current stream."""
    from vkwr_amd import capi
    from vkwr.model_executor import MixedEngine, RWKV7Config, RWKV7Model, RWKV7State
    from vkwr.model_executor.mixed import gemm_flops

    cfg = RWKV7Config.preset("7b")
    Bd, Bp, T, P = 256, 4, 512, 2048
    model = RWKV7Model(cfg, dev, seed=0)
    state = RWKV7State(cfg, P, dev, std=0.1, seed=1, layout=capi.WKV_STATE_STD)
    eng = MixedEngine(model, Bd + Bp * T, max_seqs=Bd + Bp)
    g = torch.Generator().manual_seed(5)
    dec = (torch.randint(0, cfg.vocab, (Bd,), generator=g).to(torch.int32).to(dev),
           torch.arange(0, Bd, dtype=torch.int32).to(dev))
    pre = [(torch.randint(0, cfg.vocab, (Bp, T), generator=g).to(torch.int32).to(dev),
            torch.arange(Bd, Bd + Bp, dtype=torch.int32).to(dev))]
    for _ in range(warmup):
        eng.step(state, decode=dec, prefill=pre)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(steps):
        eng.step(state, decode=dec, prefill=pre)
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / steps
    rows = Bd + Bp * T
    tflops = gemm_flops(cfg, rows, Bd + Bp) / (ms * 1e-3) / 1e12
    del eng, state, model
    torch.cuda.empty_cache()
    return {
        "workload": "RWKV-7 7B shape (BASELINE config 4): L=32, C=4096, H=64, F=16384, ranks w/a/v/g "
                    "128/128/96/480, V=65536; one continuous-batching step = 256 decode rows + 4 prefill "
                    "chunks x 512 tokens (2304 GEMM rows), 2048-slot fp32 state pool, random fp16 weights",
        "ms_per_step": round(ms, 3),
        "steps": steps,
        "rows_per_step": rows,
        "tokens_per_s": round(rows / (ms * 1e-3), 1),
        "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(tflops / 2500.0, 4),
                     "flops_per_step": gemm_flops(cfg, rows, Bd + Bp)},
        "gemm_path": "vkwr_gemm_f16 large-M path (256x256 or 192x256 tiles, k 64 per LDS-DMA stage; last round "
                     "split in equal k-parts or layered), rank-out adapters included (ranks zero-padded to "
                     "multiples of 64)",
        "wkv_path": "prefill chunks: chunked MFMA kernel; decode rows: LDS-free step kernel on a second stream "
                    "beside it",
        "timing": "eager launches, HIP events around the timed steps (the side stream joins the timed one)",
    }


def gemm_7b_shapes(dev, calls=10, warmup=3):
    """The large-M GEMM kernel (vkwr_gemm_f16) against torch.mm (hipBLASLt) on the GEMM
    shapes of one 7B mixed step (2304 rows; the head over 260), plain epilogue, random fp16
    operands.  torch.mm gets the weight as a contiguous [K, N] matrix (no transposed view),
    this kernel the nn.Linear [N, K] weight.  Each form: `calls` calls captured into one
    HIP graph, replayed once after an untimed replay; HIP events on the replay stream."""
    from vkwr_amd import capi

    g = torch.Generator(device=dev).manual_seed(13)
    stream = torch.cuda.Stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        gr = capture(lambda i: fn(), calls, stream)
        gr.replay()
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            ev0.record(stream)
            gr.replay()
            ev1.record(stream)
        torch.cuda.synchronize()
        del gr
        return ev0.elapsed_time(ev1) / calls * 1e3  # us

    R = 2304
    shapes = [("r/k/v + rank-in inputs", R, 3 * 4096 + 896, 4096), ("FFN key", R, 16384, 4096),
              ("FFN value", R, 4096, 16384), ("o projection", R, 4096, 4096), ("head", 260, 65536, 4096),
              ("rank-out w2 (K 128)", R, 4096, 128), ("rank-out g2 (K 512)", R, 4096, 512)]
    out = {}
    for name, M, N, K in shapes:
        a = torch.randn(M, K, device=dev, generator=g).half()
        w = (torch.randn(N, K, device=dev, generator=g) * 0.02).half()
        wt = w.t().contiguous()
        c = torch.empty(M, N, dtype=torch.float16, device=dev)
        c2 = torch.empty(M, N, dtype=torch.float16, device=dev)
        probs = [capi.gemm_problem(a, w, c)]
        ws = torch.empty(max(capi.gemm_workspace_bytes(probs), 1), dtype=torch.uint8, device=dev)
        us = timed(lambda: capi.gemm(probs, ws))
        us_lib = timed(lambda: torch.mm(a, wt, out=c2))
        fl = 2 * M * N * K
        out[name] = {"M": M, "N": N, "K": K, "us": round(us, 2), "TFLOP/s": round(fl / us / 1e6, 1),
                     "hipblaslt_us": round(us_lib, 2), "hipblaslt_TFLOP/s": round(fl / us_lib / 1e6, 1),
                     "vs_hipblaslt": round(us / us_lib, 3)}
        del a, w, wt, c, c2, ws
    torch.cuda.empty_cache()
    return {"shapes": out,
            "timing": "each form's calls captured into one HIP graph; HIP events on the replay stream, mean per call",
            "note": "torch.mm in fp16 dispatches to hipBLASLt on this image; weights [K, N] contiguous for it"}


def cpu_baseline(target_s):
    """Config 1 on the host cores: the oracle (C restatement, OpenMP over heads), bounded sample."""
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


def cpu_baseline_prefill(reps=5):
    """Config 2 on the host cores: the C oracle (OpenMP over the 256 (sequence, head) chains),
    B=8 x T=1024 x H=32 through the slot-pool entry (gather, 1024 tokens, scatter) on a
    512-slot pool, inputs drawn as in config 0; one untimed call, then the median of `reps`."""
    import numpy as np

    from oracle import oracle as orc
    from tests.wkv_inputs import make_state, make_wkv_inputs

    Bp, Tp = 8, 1024
    cores = len(os.sched_getaffinity(0))
    orc.set_threads(cores)
    pool = make_state(P_SLOTS, H, seed=2)
    slots = np.random.default_rng(2).permutation(P_SLOTS)[:Bp]
    ins = make_wkv_inputs(Bp, Tp, H, seed=2)
    orc.wkv_fp32_slots(Bp, Tp, C, H, pool, slots, *ins)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        orc.wkv_fp32_slots(Bp, Tp, C, H, pool, slots, *ins)
        times.append(time.perf_counter() - t0)
    t = sorted(times)[len(times) // 2]
    nbytes = 7 * Bp * Tp * C * 2 + 2 * Bp * H * HEAD * HEAD * 4 + Bp * 4
    return {
        "value": round(Bp * Tp / t, 1),
        "unit": "tokens/s",
        "GB/s": round(nbytes / t / 1e9, 3),
        "cores": cores,
        "kind": "port",
        "sample": f"config 2 whole (B=8, T=1024, H=32, one call = 8192 tokens), median of {reps} calls "
                  f"after one untimed: {t * 1e3:.1f} ms/call",
    }


def cpu_model_copy(model):
    """The decode model's weights as float32 host tensors, in the shape the float32
    composition (oracle.model_ref.decode_step) reads."""
    import types

    f = lambda t: t.float().cpu()  # noqa: E731
    return types.SimpleNamespace(cfg=model.cfg, layers=[{k: f(v) for k, v in L.items()} for L in model.layers],
                                 emb=f(model.emb), ln_out_w=f(model.ln_out_w), ln_out_b=f(model.ln_out_b),
                                 head=f(model.head))


def cpu_baseline_decode(cpu_model, steps=3):
    """Config 3 on the host cores: the float32 torch composition of the restated ops
    (oracle.model_ref.decode_step, round_fp16=False) for 128 sequences at T=1, weights and
    states in host memory, torch.set_num_threads(cores); one untimed step, then the median
    of `steps`."""
    from oracle import model_ref

    cfg = cpu_model.cfg
    B = 128
    cores = len(os.sched_getaffinity(0))
    prev = torch.get_num_threads()
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(7)
    wkv = torch.randn(cfg.n_layer, B, cfg.n_head, HEAD, HEAD, generator=g) * 0.1
    att = torch.zeros(cfg.n_layer, B, cfg.n_embd)
    ffn = torch.zeros(cfg.n_layer, B, cfg.n_embd)
    tokens = torch.randint(0, cfg.vocab, (B,), generator=g)
    slots = torch.arange(B)
    times = []
    with torch.no_grad():
        for i in range(steps + 1):
            t0 = time.perf_counter()
            model_ref.decode_step(cpu_model, wkv, att, ffn, tokens, slots, round_fp16=False)
            if i:
                times.append(time.perf_counter() - t0)
    torch.set_num_threads(prev)
    t = sorted(times)[len(times) // 2]
    return {
        "value": round(B / t, 1),
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": f"config 3 (1.5B shape, bs=128, T=1): {steps} float32 decode steps on the host after one "
                  f"untimed, median {t * 1e3:.0f} ms/step (torch CPU, {cores} threads)",
    }


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the WKV path shards by sequence with no communication between GPUs)", file=sys.stderr)
        sys.exit(2)
    assert torch.cuda.is_available(), "no GPU visible"
    import vkwr  # noqa: F401
    from vkwr._ops.v1 import v1_wkv_ops as ops

    dev = torch.device("cuda:0")
    if args.only:
        run = {"decode": lambda: model_decode(dev, args.model_steps, frag=not args.rowmajor_gemm, eager=args.eager,
                                              op_steps=0 if args.eager else args.model_steps),
               "prefill": lambda: prefill_c2(dev, args.prefill_calls),
               "serve": lambda: serve_mixed_7b(dev, args.serve_steps),
               "sampling": lambda: sampling_bs128(dev, args.sampling_calls),
               "ops": lambda: ops_small_m(dev, args.ops_calls),
               "fp16": lambda: wkv_fp16_family(dev, args.fp16_steps),
               "gemm7b": lambda: gemm_7b_shapes(dev)}.get(args.only)
        if run is None:  # "c1": the config-1 step alone (the sections below are skipped)
            args.model_steps = args.prefill_calls = args.serve_steps = 0
            args.sampling_calls = args.ops_calls = args.fp16_steps = 0
            args.no_cpu_baseline = True
    if args.only and args.only != "c1":
        copy_calibration(dev)  # a reference dispatch of known size for counter runs
        print(json.dumps({args.only: run()}), flush=True)
        return
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

    copy_calibration(dev)
    for i in range(W):
        step(K + i)
    torch.cuda.synchronize()

    stream = torch.cuda.Stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    variants = {}
    if args.eager:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        with torch.cuda.stream(stream):
            ev0.record(stream)
            for i in range(K):
                step(i)
            ev1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ms_per_step = ev0.elapsed_time(ev1) / K
    else:
        graph = capture(step, K, stream)
        graph.replay()  # one untimed replay (first replay uploads the graph)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        with torch.cuda.stream(stream):
            ev0.record(stream)
            graph.replay()
            ev1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ms_per_step = ev0.elapsed_time(ev1) / K
        del graph

        def timed_graph(fn, n):
            g = capture(fn, n, stream)
            g.replay()
            torch.cuda.synchronize()
            with torch.cuda.stream(stream):
                ev0.record(stream)
                g.replay()
                ev1.record(stream)
            torch.cuda.synchronize()
            return ev0.elapsed_time(ev1) / n

        # (1) 4 disjoint 128-slot sets of the same 512-slot pool cycled (256 MiB touched).
        sets = [perm[i * B_ACTIVE:(i + 1) * B_ACTIVE].to(torch.int32).to(dev) for i in range(4)]
        kc = min(K, 400)
        ms_rot = timed_graph(lambda i: step(i, sets[i % 4]), kc)
        variants["rotating_4_slot_sets"] = {
            "ms_per_step": round(ms_rot, 5), "GB/s": round(STEP_BYTES / (ms_rot * 1e-3) / 1e9, 2),
            "note": "4 disjoint 128-slot sets of the 512-slot pool cycled (256 MiB touched)"}
        # (2) cold: a 2048-slot pool (1 GiB, 4x the 256 MB Infinity Cache), 16 disjoint sets cycled.
        del sets
        big = torch.empty(COLD_SLOTS, H, HEAD, HEAD, dtype=torch.float32, device=dev).normal_(0.0, 0.1)
        bperm = torch.randperm(COLD_SLOTS, generator=gen)
        bsets = [bperm[i * B_ACTIVE:(i + 1) * B_ACTIVE].to(torch.int32).to(dev)
                 for i in range(COLD_SLOTS // B_ACTIVE)]

        def cold_step(i):
            x = inputs[i]
            op(B_ACTIVE, 1, C, H, big, bsets[i % len(bsets)], x[0], x[1], x[2], x[3], x[4], x[5], y)

        ms_cold = timed_graph(cold_step, kc)
        variants["cold_1GiB_pool"] = {
            "ms_per_step": round(ms_cold, 5), "GB/s": round(STEP_BYTES / (ms_cold * 1e-3) / 1e9, 2),
            "frac_of_peak": round(STEP_BYTES / (ms_cold * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "note": f"{COLD_SLOTS}-slot pool (1 GiB), {len(bsets)} disjoint 128-slot sets cycled: "
                    "every step's state comes from HBM, not the Infinity Cache"}
        del big
        # (3) references for the cold case, the same bytes per step through torch's elementwise
        # kernels, 16 regions of 64 MiB cycled so that each step's bytes come from HBM: a
        # streaming copy from one 1 GiB buffer into another, and an in-place rewrite.
        n64 = B_ACTIVE * H * HEAD * HEAD
        src = torch.empty(16 * n64, dtype=torch.float32, device=dev).normal_(0.0, 0.1)
        dst = torch.empty_like(src)
        ms_copy = timed_graph(lambda i: dst[(i % 16) * n64:(i % 16 + 1) * n64].copy_(
            src[(i % 16) * n64:(i % 16 + 1) * n64]), kc)
        ms_inpl = timed_graph(lambda i: src[(i % 16) * n64:(i % 16 + 1) * n64].mul_(0.5), kc)
        for name, ms_ref in (("ref_stream_copy_64MiB_cold", ms_copy), ("ref_inplace_rewrite_64MiB_cold", ms_inpl)):
            variants[name] = {"ms_per_step": round(ms_ref, 5),
                              "GB/s": round(2 * n64 * 4 / (ms_ref * 1e-3) / 1e9, 2),
                              "note": "64 MiB read + 64 MiB written per step, 16 regions of two 1 GiB buffers "
                                      "cycled (torch copy_ / mul_)"}
        del src, dst
    variants["wall_s_timed_region"] = round(wall, 4)
    log("config 1 decode step done")
    gbs = STEP_BYTES / (ms_per_step * 1e-3) / 1e9

    traffic = read_traffic()
    cold = variants.get("cold_1GiB_pool")
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
                   "state": "fp32", "io": "fp16", "timing": ("eager launches" if args.eager else "HIP graph of K steps") + ", HIP events on the launch stream"},
        "tokens_per_s": round(B_ACTIVE / (ms_per_step * 1e-3), 1),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "bytes_per_launch": STEP_BYTES,
                     "frac_cold_1GiB_pool": cold["frac_of_peak"] if cold else None,
                     "note": "frac: the config as specified, whose 64 MiB of active state stays in the 256 MB "
                             "Infinity Cache between steps; frac_cold_1GiB_pool: the same step over a 1 GiB pool "
                             "whose every step's state comes from HBM. traffic: FETCH_SIZE + WRITE_SIZE bytes per "
                             "launch (rocprofv3, scaled by a plain copy of known size); these count L2-to-fabric "
                             "requests, Infinity Cache hits included, so they show no re-reads, not HBM bytes"},
        "variants": variants,
        "cpu_baseline": None,
    }
    keep = [] if not args.no_cpu_baseline else None

    def section(fn, done):
        """Runs one secondary section; a Python-level failure (out of memory, a failed check) is
        recorded in its place and the line is still printed."""
        try:
            out = fn()
        except Exception as e:  # noqa: BLE001
            traceback.print_exc()
            out = {"error": f"{type(e).__name__}: {e}"}
        torch.cuda.empty_cache()
        log(done)
        return out

    if args.model_steps > 0 and not args.eager:
        del inputs
        torch.cuda.empty_cache()
        result["decode_1p5b_bs128"] = section(
            lambda: model_decode(dev, args.model_steps, frag=not args.rowmajor_gemm, keep_cpu_model=keep,
                                 op_steps=args.model_steps), "config 3 decode step done")
    if args.prefill_calls > 0 and not args.eager:
        result["prefill_c2"] = section(lambda: prefill_c2(dev, args.prefill_calls), "config 2 prefill done")
    if args.fp16_steps > 0 and not args.eager:
        result["wkv_fp16_family"] = section(lambda: wkv_fp16_family(dev, args.fp16_steps),
                                            "fp16-state WKV done")
    if args.serve_steps > 0 and not args.eager:
        def serve():
            out = serve_mixed_7b(dev, args.serve_steps)
            out["gemm_shapes_vs_hipblaslt"] = gemm_7b_shapes(dev)
            return out
        result["serve_mixed_7b"] = section(serve, "config 4 mixed step done")
    if args.sampling_calls > 0 and not args.eager:
        result["sampling_bs128"] = section(lambda: sampling_bs128(dev, args.sampling_calls),
                                           "sampling done")
    if args.ops_calls > 0 and not args.eager:
        result["ops_small_m"] = section(lambda: ops_small_m(dev, args.ops_calls), "op-surface GEMMs done")
    if not args.no_cpu_baseline:
        cb = cpu_baseline(args.cpu_seconds)
        log("CPU baseline, config 1 done")
        per = {"config1_decode_step": dict(cb)}
        if "error" not in result.get("prefill_c2", {"error": None}):
            per["config2_prefill"] = result["prefill_c2"]["cpu_baseline"] = section(
                cpu_baseline_prefill, "CPU baseline, config 2 done")
        if keep:
            per["config3_decode_1p5b"] = result["decode_1p5b_bs128"]["cpu_baseline"] = section(
                lambda: cpu_baseline_decode(keep.pop()), "CPU baseline, config 3 done")
        cb["per_config"] = per
        result["cpu_baseline"] = cb
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
