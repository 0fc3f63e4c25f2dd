#!/usr/bin/env python3
"""Benchmark of the BDH recurrent-attention forward path on one MI355X.

Headline (``value``): chunked prefill of one BDH layer, BASELINE config 2:
B=8, nh=4, T=512, N=8192, D=256, chunk 128, bf16 inputs / fp32 accumulate,
RoPE (theta 65536) fused, tokens/s = B*T / step time.  A step is one call of
the RoPE-fused recurrent forward over the whole batch (inputs resident in HBM).

Also reported (``decode``): BASELINE config 3, 256 decode steps of B=64
streams after a 1024-token prefill, fp32 rho, tokens/s = B / step time, with
its HBM roofline.

Roofline (algorithmic work; the bound kernel is timed live with HIP events):
  prefill FLOP/step = B*nh*T*(4*N*D + (C-1)*(N+D))          vs 2.5 PFLOP/s bf16
  decode  bytes/step = sum_streams (4N + 4D + 2*|A|*4D + 4D)  vs 8 TB/s HBM
with |A| the exact active-row count of each stream at that step.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

METRIC = "prefill & decode tokens/s per BDH layer (D=256,n=32K); % MFMA / HBM roofline"
PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA
PEAK_F32_TFLOPS = 157.3       # MI355X dense fp32 MFMA
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E
SEED = 20260729

# HBM-side bytes per launch of each leg's measured unit, from rocprofv3
# FETCH_SIZE and WRITE_SIZE runs of this script (one counter per run), each
# scaled by what the counter reads for a 1 GiB device copy (--only copy):
# FETCH_SIZE x 2.0, WRITE_SIZE x 1.0.  Commands and per-kernel figures:
# profiles/prefill_c2_traffic.txt, profiles/decode_c3_traffic.txt,
# profiles/long_prefill_c4_traffic.txt.  Counters cannot run inside this
# process, so the figures are recorded here; they change when the kernels do.
TRAFFIC_PREFILL_C2 = 1098.4e6       # one prefill_mfma_kernel launch
TRAFFIC_PREFILL_C2_PASS = 1165.7e6  # the whole C2 pass (transpose_v, prefill, ctx)
TRAFFIC_DECODE_C3 = 428.0e6         # one decode_kernel launch
TRAFFIC_LONG_C4 = 2637.0e6          # the carry and snap_wide launches of one C4 call (row chunk 512)
TRAFFIC_LONG_C4_CALL = 2834.5e6     # the whole C4 call


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20, help="timed prefill steps")
    ap.add_argument("--warmup", type=int, default=3, help="untimed prefill steps")
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--decode-warmup", type=int, default=4)
    ap.add_argument("--decode-prefill", type=int, default=1024, help="tokens prefilled into rho")
    ap.add_argument("--model-steps", type=int, default=6, help="timed C5 model forwards")
    ap.add_argument("--model-warmup", type=int, default=2, help="untimed C5 model forwards before them")
    ap.add_argument("--model-decode-steps", type=int, default=32,
                    help="timed C5 greedy decode steps")
    ap.add_argument("--only", choices=("all", "prefill", "decode", "long", "model", "model-decode",
                                       "f32", "copy", "rmw", "ceilings"),
                    default="all",
                    help="one leg only; 'copy' times a 1 GiB device copy (the calibration kernel "
                         "of the FETCH_SIZE / WRITE_SIZE counter runs); 'ceilings' (or 'rmw') "
                         "measures what the device sustains: HBM read, copy, in-place RMW and "
                         "RMW of random 1 KiB rows on a buffer the size of C3's rho, torch "
                         "copy_/add_, the bf16 MFMA rate on register operands, and hipBLASLt on "
                         "the C2 gram and state shapes")
    ap.add_argument("--long-steps", type=int, default=10, help="timed C4 prefills")
    ap.add_argument("--cpu-seconds", type=float, default=20.0,
                    help="target CPU-baseline wall time (split between prefill and decode)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    return ap.parse_args()


# --------------------------------------------------------------------------- #
def lib_fwd_call(torch, lib, plan, x, v, rope, ctx, rho, chunk=0, decay=None):
    """One RoPE-fused bf16 forward; chunk = the row chunk (rho materialised
    every `chunk` tokens, 0 = 512); decay [H] f32 on the device or None."""
    from burn_dragon_amd import _lib
    st = lib.bdh_recurrent_attention_rope_fwd(
        ctypes.byref(plan), _lib.BDH_BF16, ctypes.c_void_p(x.data_ptr()),
        ctypes.c_void_p(v.data_ptr()), None,
        ctypes.c_void_p(decay.data_ptr()) if decay is not None else None, ctypes.byref(rope),
        ctypes.c_void_p(ctx.data_ptr()), ctypes.c_void_p(rho.data_ptr()), chunk,
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    if st != 0:
        raise RuntimeError(f"prefill failed: {_lib.last_error()}")


def kernel_times(lib, kind):
    """(summed ms, launches) of the dominant kernel `kind` recorded since
    bdh_profile_kernel_timing(1): HIP events on the launch stream around each
    of its launches."""
    from burn_dragon_amd import _lib
    ms, n = ctypes.c_double(), ctypes.c_int64()
    if lib.bdh_profile_kernel_get(kind, ctypes.byref(ms), ctypes.byref(n)) != 0:
        raise RuntimeError(f"kernel timing failed: {_lib.last_error()}")
    return ms.value, n.value


def timed_kernel(torch, lib, kind, steps, call):
    """Run `call` `steps` times with kernel timing on; returns (ms per call of
    the kernel, launches per call)."""
    lib.bdh_profile_kernel_timing(1)
    for _ in range(steps):
        call()
    torch.cuda.synchronize()
    ms, n = kernel_times(lib, kind)
    lib.bdh_profile_kernel_timing(0)
    return ms / steps, n / steps


def bench_prefill(torch, args):
    from burn_dragon_amd import _lib
    B, H, T, N, D, C = 8, 4, 512, 8192, 256, 128
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(SEED + 2)
    x = torch.relu(torch.randn(B, H, T, N, generator=g, device=dev) - 1.645).to(torch.bfloat16)
    v = (torch.randn(B, 1, T, D, generator=g, device=dev) / 16).to(torch.bfloat16)
    ctx = torch.empty(B, H, T, D, device=dev, dtype=torch.float32)
    rho = torch.empty(B, H, N, D, device=dev, dtype=torch.float32)
    lib = _lib.load()
    plan = _lib.BdhRecurrentPlan(B, H, 1, T, N, D)
    rope = _lib.BdhRope(_lib.BDH_ROPE_SEQUENTIAL, 0, 0, 65536.0)
    for _ in range(args.warmup):
        lib_fwd_call(torch, lib, plan, x, v, rope, ctx, rho)
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        starts[i].record()
        lib_fwd_call(torch, lib, plan, x, v, rope, ctx, rho)
        ends[i].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    eager_ev_ms = sum(s.elapsed_time(e) for s, e in zip(starts, ends)) / args.steps
    eager_ms = wall * 1e3 / args.steps
    # The pass captured once into a HIP graph (torch.cuda.CUDAGraph) and
    # replayed: the deployment form of a fixed-shape prefill, without the
    # host launch gaps.  Every replay recomputes ctx and rho in full; the
    # replays are checked bit for bit against the eager result first.
    # The library keeps its scratch per stream and cannot grow it during a
    # capture, so the capture runs on a stream that made one eager call.
    ref_ctx, ref_rho = ctx.clone(), rho.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        lib_fwd_call(torch, lib, plan, x, v, rope, ctx, rho)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        lib_fwd_call(torch, lib, plan, x, v, rope, ctx, rho)
    for _ in range(3):
        ctx.zero_()
        rho.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        if not (torch.equal(ctx, ref_ctx) and torch.equal(rho, ref_rho)):
            raise RuntimeError("graph replay differs from the eager prefill")
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    ev_ms = e0.elapsed_time(e1) / args.steps
    del graph
    flop = B * H * T * (4 * N * D + (C - 1) * (N + D))
    pass_tflops = flop / (ev_ms * 1e-3) / 1e12
    # The dominant kernel, timed in its own loop: prefill_mfma_kernel does all
    # of the pass's algorithmic work except the intra-chunk S.V (C-1)D per
    # token, which is the context kernel's.
    k_ms, k_n = timed_kernel(torch, lib, _lib.BDH_KERNEL_PREFILL, args.steps,
                             lambda: lib_fwd_call(torch, lib, plan, x, v, rope, ctx, rho))
    k_flop = B * H * T * (4 * N * D + (C - 1) * N)
    achieved = k_flop / k_n / (k_ms / k_n * 1e-3) / 1e12
    print(f"[prefill] graph {ms:.3f} ms/step wall, {ev_ms:.3f} ms/step events, "
          f"{B * T / (ms * 1e-3) / 1e6:.2f} M tok/s, {pass_tflops:.1f} TFLOP/s per pass; "
          f"eager {eager_ms:.3f} ms wall, {eager_ev_ms:.3f} ms events; "
          f"prefill_mfma_kernel {k_ms / k_n * 1e3:.1f} us, {achieved:.1f} TFLOP/s", flush=True)
    return {
        "ms_per_step": ms, "event_ms": ev_ms, "tokens_per_s": B * T / (ms * 1e-3),
        "eager": {"ms_per_step": round(eager_ms, 4), "event_ms": round(eager_ev_ms, 4),
                  "tokens_per_s": round(B * T / (eager_ms * 1e-3), 1)},
        "flop": flop,
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": TRAFFIC_PREFILL_C2, "kernel": "prefill_mfma_kernel",
                     "kernel_avg_us": round(k_ms / k_n * 1e3, 2), "flop_per_launch": k_flop / k_n,
                     "pass": {"kernels": "transpose_v_kernel + prefill_mfma_kernel + ctx_kernel",
                              "event_ms": round(ev_ms, 4), "tflops": round(pass_tflops, 2),
                              "flop": flop, "traffic": TRAFFIC_PREFILL_C2_PASS}},
        "shape": {"B": B, "nh": H, "T": T, "N": N, "D": D, "chunk": C},
    }


def bench_long(torch, args):
    """C4: one long stream per head, T = 8192 (16 state-carry intervals at the
    automatic row chunk of 512: the state-carry launch, then one launch of
    every interval's gram and readout tiles, then the context launch)."""
    from burn_dragon_amd import _lib
    B, H, T, N, D, C = 1, 4, 8192, 8192, 256, 256
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(SEED + 4)
    x = torch.relu(torch.randn(B, H, T, N, generator=g, device=dev) - 1.645).to(torch.bfloat16)
    v = (torch.randn(B, 1, T, D, generator=g, device=dev) / 16).to(torch.bfloat16)
    ctx = torch.empty(B, H, T, D, device=dev, dtype=torch.float32)
    rho = torch.empty(B, H, N, D, device=dev, dtype=torch.float32)
    lib = _lib.load()
    plan = _lib.BdhRecurrentPlan(B, H, 1, T, N, D)
    rope = _lib.BdhRope(_lib.BDH_ROPE_SEQUENTIAL, 0, 0, 65536.0)
    for _ in range(2):
        lib_fwd_call(torch, lib, plan, x, v, rope, ctx, rho)
    torch.cuda.synchronize()
    steps = args.long_steps
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        lib_fwd_call(torch, lib, plan, x, v, rope, ctx, rho)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    # The same call at the config's row chunk of 256 (32 state intervals):
    # the result is the same up to rounding; the automatic row chunk (512)
    # writes half as many state snapshots.
    for _ in range(2):
        lib_fwd_call(torch, lib, plan, x, v, rope, ctx, rho, chunk=C)
    e0.record()
    for _ in range(steps):
        lib_fwd_call(torch, lib, plan, x, v, rope, ctx, rho, chunk=C)
    e1.record()
    torch.cuda.synchronize()
    ms_c = e0.elapsed_time(e1) / steps
    # The same call with ALiBi-style decay per head (the state-carry form with
    # decay: weighted q^T rows, the carried block scaled per interval).
    dk = torch.tensor([0.999, 0.998, 0.997, 0.996], device=dev, dtype=torch.float32)
    for _ in range(2):
        lib_fwd_call(torch, lib, plan, x, v, rope, ctx, rho, decay=dk)
    e0.record()
    for _ in range(steps):
        lib_fwd_call(torch, lib, plan, x, v, rope, ctx, rho, decay=dk)
    e1.record()
    torch.cuda.synchronize()
    ms_d = e0.elapsed_time(e1) / steps
    flop = B * H * T * (4 * N * D + (C - 1) * (N + D))
    call_tflops = flop / (ms * 1e-3) / 1e12
    # The dominant kernels: a call's state-carry launch and its gram/readout
    # launch, summed (they hold all of the call's algorithmic work but the
    # intra-chunk S.V term).
    k_ms, k_n = timed_kernel(torch, lib, _lib.BDH_KERNEL_PREFILL, steps,
                             lambda: lib_fwd_call(torch, lib, plan, x, v, rope, ctx, rho))
    k_flop = B * H * T * (4 * N * D + (C - 1) * N)
    achieved = k_flop / (k_ms * 1e-3) / 1e12
    print(f"[long] {ms:.3f} ms/prefill, {B * T / (ms * 1e-3) / 1e6:.2f} M tok/s, "
          f"{call_tflops:.1f} TFLOP/s per call; carry + snap_wide kernels {k_n:.0f} launches, "
          f"{k_ms:.3f} ms, {achieved:.1f} TFLOP/s; at row chunk {C}: {ms_c:.3f} ms; with decay: "
          f"{ms_d:.3f} ms", flush=True)
    return {"metric": "C4 long-context prefill tokens/s per BDH layer", "value": B * T / (ms * 1e-3),
            "unit": "tokens/s", "ms_per_prefill": ms, "steps": steps,
            "config": {"workload": "C4 long prefill, one BDH layer: B1 nh4 T8192 N8192 D256, "
                                   "bf16 in / fp32 acc, RoPE fused; automatic row chunk (rho "
                                   "snapshots every 512 tokens), credited at the config's "
                                   f"chunk {C}"},
            "at_config_chunk": {"chunk": C, "ms_per_prefill": round(ms_c, 4),
                                "tokens_per_s": round(B * T / (ms_c * 1e-3), 1)},
            "with_decay": {"decay": [0.999, 0.998, 0.997, 0.996], "ms_per_prefill": round(ms_d, 4),
                           "tokens_per_s": round(B * T / (ms_d * 1e-3), 1)},
            "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                         "traffic": TRAFFIC_LONG_C4,
                         "kernel": f"prefill_carry_kernel + snap_wide_kernel, {k_n:.0f} launches "
                                   "per call (summed)",
                         "kernel_ms_per_call": round(k_ms, 4), "flop_per_call": k_flop,
                         "call": {"tflops": round(call_tflops, 2), "flop": flop, "traffic": TRAFFIC_LONG_C4_CALL}}}


def bench_decode(torch, args):
    import burn_dragon_amd as bd
    from burn_dragon_amd import _lib, rope as rp
    B, H, N, D = 64, 4, 8192, 256
    P = args.decode_prefill
    K = args.decode_steps
    W = args.decode_warmup
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(SEED + 3)
    # rho pre-filled by a P-token synthetic prefill (untimed), bf16 MFMA path.
    rho = torch.empty(B, H, N, D, device=dev, dtype=torch.float32)
    lib = _lib.load()
    step_b = 16
    for b0 in range(0, B, step_b):
        xp = torch.relu(torch.randn(step_b, H, P, N, generator=g, device=dev) - 1.645).to(torch.bfloat16)
        vp = (torch.randn(step_b, 1, P, D, generator=g, device=dev) / 16).to(torch.bfloat16)
        ctxp = torch.empty(step_b, H, P, D, device=dev, dtype=torch.float32)
        plan = _lib.BdhRecurrentPlan(step_b, H, 1, P, N, D)
        rope = _lib.BdhRope(_lib.BDH_ROPE_SEQUENTIAL, 0, 0, 65536.0)
        lib_fwd_call(torch, lib, plan, xp, vp, rope, ctxp, rho[b0:b0 + step_b])
        del xp, vp, ctxp
    torch.cuda.synchronize()
    xs = torch.relu(torch.randn(W + K, B, H, N, generator=g, device=dev) - 1.645)
    vs = torch.randn(W + K, B, 1, D, generator=g, device=dev) / 16
    a = torch.empty(B, H, D, device=dev, dtype=torch.float32)
    rope = _lib.BdhRope(_lib.BDH_ROPE_SEQUENTIAL, 0, 0, 65536.0)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def step(i):
        rope.pos0 = P + i
        st = lib.bdh_decode_step(B, H, 1, N, D, ctypes.c_void_p(xs[i].data_ptr()),
                                 ctypes.c_void_p(vs[i].data_ptr()), ctypes.c_void_p(rho.data_ptr()),
                                 None, ctypes.byref(rope), ctypes.c_void_p(a.data_ptr()), None, None,
                                 stream)
        if st != 0:
            raise RuntimeError(f"decode failed: {_lib.last_error()}")

    for i in range(W):
        step(i)
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(K)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(K)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(K):
        starts[k].record()
        step(W + k)
        ends[k].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ev = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    ev_ms = sum(ev) / K
    # exact active rows per step -> algorithmic bytes
    freqs = torch.from_numpy(rp.rope_freqs(N)).to(dev)
    active = 0
    for k in range(K):
        active += int(rp.active_rows_mask(xs[W + k], P + W + k, freqs).sum().item())
    S = B * H
    bytes_total = K * S * (4 * N + 4 * D + 4 * D) + active * 2 * 4 * D
    bytes_per_step = bytes_total / K
    # The kernel alone, timed in its own loop over the same inputs and
    # positions (the same active rows, so the same algorithmic bytes).
    it = iter(range(W, W + K))
    k_ms, k_n = timed_kernel(torch, lib, _lib.BDH_KERNEL_DECODE, K, lambda: step(next(it)))
    achieved = bytes_per_step / (k_ms / k_n * 1e-3) / 1e9
    ms = wall * 1e3 / K
    frac_active = active / (K * S * N)
    print(f"[decode] {ms:.4f} ms/step wall, {ev_ms:.4f} ms/step events, "
          f"{B / (ms * 1e-3) / 1e6:.3f} M tok/s, decode_kernel {k_ms / k_n * 1e3:.1f} us, "
          f"{achieved:.0f} GB/s, active {frac_active:.4f}", flush=True)
    del xs, vs, rho
    return {
        "value": B / (ms * 1e-3), "unit": "tokens/s", "steps": K, "warmup": W,
        "ms_per_step": ms, "event_ms": ev_ms,
        "config": {"workload": "C3 decode, one BDH layer: B64 nh4 N8192 D256, fp32 rho "
                   f"[64,4,8192,256] prefilled by {P} tokens, {K} steps, RoPE at the step position"},
        "active_fraction": round(frac_active, 5),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": TRAFFIC_DECODE_C3,
                     "kernel": "decode_kernel", "kernel_avg_us": round(k_ms / k_n * 1e3, 2),
                     "bytes_per_launch": round(bytes_per_step)},
    }


# --------------------------------------------------------------------------- #
def _cpu_model() -> str:
    """Model name of the host CPU with its family / model / stepping numbers
    (a virtual machine may report only a generic name)."""
    info = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if ":" in line:
                    k, v = (t.strip() for t in line.split(":", 1))
                    if k in ("model name", "cpu family", "model", "stepping") and k not in info:
                        info[k] = v
                if not line.strip() and info:
                    break
    except OSError:
        pass
    name = info.get("model name", "unknown")
    ids = ", ".join(f"{k} {info[k]}" for k in ("cpu family", "model", "stepping") if k in info)
    return f"{name} ({ids}; {os.cpu_count()} logical CPUs visible)" if ids else \
        f"{name} ({os.cpu_count()} logical CPUs visible)"


def cpu_baseline_prefill(target_s: float):
    """Reference CPU path restated (oracle, test infrastructure): RoPE in the
    reference's f32 op order, then the NdArray recurrence op sequence with
    [N, D] temporaries, fp32, OpenMP over the 32 (b, h) streams, on a sample of
    the C2 workload's first tokens."""
    import numpy as np
    from oracle import oracle as O
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or min(16, os.cpu_count() or 1)
    B, H, N, D = 8, 4, 8192, 256
    rng = np.random.default_rng(SEED + 2)
    # Grow the token count until one pass takes a measurable time (the whole
    # C2 sequence, T = 512, takes a few seconds on 16 cores), then repeat
    # passes until about half the target wall time is spent.
    T = 4
    while True:
        x = np.maximum(rng.standard_normal((B, H, T, N), dtype=np.float32) - np.float32(1.645), 0)
        v = (rng.standard_normal((B, 1, T, D), dtype=np.float32) / np.float32(16)).astype(np.float32)
        t0 = time.perf_counter()
        q = O.rope_rotate(x, pos0=0)
        O.ndarray_recurrent_f32(q, v, threads=threads)
        secs = time.perf_counter() - t0
        if secs >= target_s / 8 or T >= 512:
            break
        T = min(512, T * 4)
    passes, total = 1, secs
    while total < target_s / 2:
        t0 = time.perf_counter()
        q = O.rope_rotate(x, pos0=0)
        O.ndarray_recurrent_f32(q, v, threads=threads)
        total += time.perf_counter() - t0
        passes += 1
    # The same op sequence on one thread: one batch row (4 head streams) over
    # an eighth of the tokens, so it takes about a quarter of the run above.
    T1 = max(4, T // 8)
    t0 = time.perf_counter()
    q1 = O.rope_rotate(x[:1, :, :T1], pos0=0)
    O.ndarray_recurrent_f32(q1, v[:1, :, :T1], threads=1)
    secs1 = time.perf_counter() - t0
    return {"value": round(B * T * passes / total, 1), "unit": "tokens/s", "cores": threads,
            "kind": "port", "host": _cpu_model(), "nproc": _nproc(),
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS"),
            "sample": f"C2 shapes (B8 nh4 N8192 D256), first {T} tokens x {passes} passes, fp32, "
                      f"RoPE + NdArray op-sequence recurrence (linear.rs:43-57) restated in C, "
                      f"{total:.2f} s wall",
            "one_thread": {"value": round(T1 / secs1, 2), "unit": "tokens/s", "cores": 1,
                           "sample": f"C2 shapes, batch row 0 (4 head streams), first {T1} tokens, "
                                     f"same op sequence, {secs1:.2f} s wall"},
            "c1_full": cpu_c1_full(threads)}


def _nproc() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def cpu_c1_full(threads: int):
    """BASELINE config 1 timed in full on the CPU (B1 nh4 T256 N1024 D64, fp32,
    V ~ N(0,1), RoPE theta 65536): the NdArray recurrent op sequence
    (linear.rs:43-57) and the dense-score form (linear.rs:241, 321), each on
    `threads` threads and on one (the four (b, h) streams bound the useful
    thread count at 4)."""
    import numpy as np
    from oracle import oracle as O
    B, H, T, N, D = 1, 4, 256, 1024, 64
    rng = np.random.default_rng(SEED + 1)
    x = np.maximum(rng.standard_normal((B, H, T, N), dtype=np.float32) - np.float32(1.645), 0)
    v = rng.standard_normal((B, 1, T, D), dtype=np.float32)
    out = {"shape": "B1 nh4 T256 N1024 D64, fp32"}
    for th in (threads, 1):
        t0 = time.perf_counter()
        q = O.rope_rotate(x, pos0=0)
        t_rope = time.perf_counter() - t0
        _, _, t_rec = O.ndarray_recurrent_f32(q, v, threads=th)
        _, t_dense = O.ndarray_dense_f32(q, v, threads=th)
        out[f"threads_{th}"] = {"recurrent_form_ms": round((t_rope + t_rec) * 1e3, 2),
                                "dense_score_form_ms": round((t_rope + t_dense) * 1e3, 2),
                                "recurrent_tokens_per_s": round(B * T / (t_rope + t_rec), 1)}
    return out


def cpu_baseline_decode(target_s: float):
    import numpy as np
    from oracle import oracle as O
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or min(16, os.cpu_count() or 1)
    B, H, N, D = 4, 4, 8192, 256
    rng = np.random.default_rng(SEED + 3)
    rho = (rng.standard_normal((B, H, N, D), dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    steps = 0
    t_total = 0.0
    while t_total < target_s / 2 and steps < 4096:
        x = np.maximum(rng.standard_normal((B, H, 1, N), dtype=np.float32) - np.float32(1.645), 0)
        v = (rng.standard_normal((B, 1, 1, D), dtype=np.float32) / np.float32(16)).astype(np.float32)
        t0 = time.perf_counter()
        q = O.rope_rotate(x, pos0=1024 + steps)
        _, rho, _ = O.ndarray_recurrent_f32(q, v, rho, threads=threads)
        t_total += time.perf_counter() - t0
        steps += 1
    return {"value": round(B * steps / t_total, 1), "unit": "tokens/s", "cores": threads,
            "kind": "port", "host": _cpu_model(), "nproc": _nproc(),
            "sample": f"C3 shapes with B={B} (16 streams), {steps} steps, fp32, RoPE + NdArray "
                      f"op-sequence step over all N*D of rho, {t_total:.2f} s wall"}


def bench_model(torch, args):
    """6-layer BDH forward over a byte vocabulary, B16 T1024
    D256 nh4 N8192, low-rank weights shared across layers (std 0.02 random
    init), uniform random tokens: embed + LN, 6 x layer body (bf16 MFMA
    GEMMs, RoPE-fused attention), logits."""
    import burn_dragon_amd as bd
    B, T, V, D, H, N, L = 16, 1024, 256, 256, 4, 8192, 6
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(SEED + 5)
    std = 0.02
    w = bd.pack_model(torch.randn(V, D, generator=g, device=dev) * std,
                      torch.randn(1, H, D, N, generator=g, device=dev) * std,
                      torch.randn(1, H, D, N, generator=g, device=dev) * std,
                      torch.randn(H * N, D, generator=g, device=dev) * std,
                      torch.randn(D, V, generator=g, device=dev) * std, L)
    if w is None:
        raise RuntimeError("model weights unsupported")
    tokens = torch.randint(0, V, (B, T), generator=g, device=dev, dtype=torch.int32)
    for _ in range(max(1, args.model_warmup)):
        assert bd.model_forward_logits(tokens, w, position=0) is not None
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    steps = args.model_steps
    e0.record()
    for _ in range(steps):
        bd.model_forward_logits(tokens, w, position=0)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    M, HN, C = B * T, H * N, 128
    per_layer = 3 * 2 * M * D * HN + B * H * T * (4 * N * D + (C - 1) * (N + D))
    flop = L * per_layer + 2 * M * D * V
    achieved = flop / (ms * 1e-3) / 1e12
    print(f"[model] {ms:.2f} ms/forward, {M / (ms * 1e-3) / 1e6:.2f} M tok/s, "
          f"{achieved:.1f} TFLOP/s", flush=True)
    return {"metric": "C5 6-layer BDH forward tokens/s", "value": M / (ms * 1e-3),
            "unit": "tokens/s", "ms_per_forward": ms, "steps": steps, "warmup": max(1, args.model_warmup),
            "config": {"workload": "C5 6-layer BDH forward, byte vocabulary: B16 T1024 D256 nh4 "
                                   "N8192, shared low-rank weights std 0.02, bf16 MFMA / fp32 acc, "
                                   "RoPE fused, random tokens"},
            "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                         "traffic": None, "flop_per_launch": flop}}


def bench_model_decode(torch, args):
    """Generation with the C5 model: a 1024-token prompt through the stateful
    forward (each layer's rho kept), then greedy T = 1 steps, every layer
    taking the sparse decode step on its own rho (generation.rs:458,
    dragon.rs:1749-1808).  The next token is the device-side argmax of the
    logits: no host sync inside the timed steps."""
    import burn_dragon_amd as bd
    B, T, V, D, H, N, L = 16, 1024, 256, 256, 4, 8192, 6
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(SEED + 6)
    std = 0.02
    w = bd.pack_model(torch.randn(V, D, generator=g, device=dev) * std,
                      torch.randn(1, H, D, N, generator=g, device=dev) * std,
                      torch.randn(1, H, D, N, generator=g, device=dev) * std,
                      torch.randn(H * N, D, generator=g, device=dev) * std,
                      torch.randn(D, V, generator=g, device=dev) * std, L)
    if w is None:
        raise RuntimeError("model weights unsupported")
    prompt = torch.randint(0, V, (B, T), generator=g, device=dev, dtype=torch.int32)
    state = bd.new_model_state(w, B, dev)
    logits = bd.model_forward_logits(prompt, w, state=state)
    if logits is None:
        raise RuntimeError("stateful model forward failed")

    def step(lg):
        tok = lg[:, -1].argmax(-1).to(torch.int32).unsqueeze(1)
        out = bd.model_forward_logits(tok, w, state=state)
        if out is None:
            raise RuntimeError("model decode step failed")
        return out

    for _ in range(args.decode_warmup):
        logits = step(logits)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    steps = args.model_decode_steps
    e0.record()
    for _ in range(steps):
        logits = step(logits)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    print(f"[model-decode] {ms:.3f} ms/token step, {B / (ms * 1e-3):.0f} tok/s "
          f"(B{B}, {L} layers, after a {T}-token prompt)", flush=True)
    return {"metric": "C5 6-layer BDH greedy decode tokens/s", "value": B / (ms * 1e-3),
            "unit": "tokens/s", "ms_per_token_step": ms, "steps": steps,
            "config": {"workload": f"C5 model decode: B{B}, {T}-token prompt, then T = 1 steps "
                                   "with every layer's rho carried (sparse decode step), greedy "
                                   "device-side argmax"}}


def bench_copy(torch):
    """A plain 1 GiB device-to-device copy: the known-size kernel against which
    the FETCH_SIZE / WRITE_SIZE counters are scaled (a copy reads and writes
    exactly 1 GiB)."""
    n = 1 << 28
    a = torch.ones(n, device="cuda", dtype=torch.float32)
    b = torch.empty_like(a)
    for _ in range(2):
        b.copy_(a)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(5):
        b.copy_(a)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / 5
    print(json.dumps({"copy_bytes": 4 * n, "ms": round(ms, 4),
                      "read_plus_write_GBs": round(2 * 4 * n / (ms * 1e-3) / 1e9, 1)}), flush=True)


def bench_f32(torch, args):
    """The fp32 path, the one an unchanged f32 Burn model reaches (the
    reference's fused op accepts F32 only, forward_runtime.rs:69-96), through
    bdh_recurrent_attention_rope_fwd: BASELINE config 1 in full (B1 nh4 T256
    N1024 D64, V ~ N(0,1)) and the C2 shape in fp32.  FLOP per call are the
    recurrent form's 4*N*D per token and stream (the figure BASELINE quotes for
    C1 as 0.268 GFLOP)."""
    from burn_dragon_amd import _lib
    lib = _lib.load()
    dev = torch.device("cuda")
    out = {}
    for name, (B, H, T, N, D, vscale) in (("c1", (1, 4, 256, 1024, 64, 1.0)),
                                          ("c2_shape", (8, 4, 512, 8192, 256, 1.0 / 16))):
        g = torch.Generator(device=dev).manual_seed(SEED + 11)
        x = torch.relu(torch.randn(B, H, T, N, generator=g, device=dev) - 1.645)
        v = torch.randn(B, 1, T, D, generator=g, device=dev) * vscale
        ctx = torch.empty(B, H, T, D, device=dev)
        rho = torch.empty(B, H, N, D, device=dev)
        plan = _lib.BdhRecurrentPlan(B, H, 1, T, N, D)
        rope = _lib.BdhRope(_lib.BDH_ROPE_SEQUENTIAL, 0, 0, 65536.0)
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

        def call():
            st = lib.bdh_recurrent_attention_rope_fwd(
                ctypes.byref(plan), _lib.BDH_F32, ctypes.c_void_p(x.data_ptr()),
                ctypes.c_void_p(v.data_ptr()), None, None, ctypes.byref(rope),
                ctypes.c_void_p(ctx.data_ptr()), ctypes.c_void_p(rho.data_ptr()), 0, stream)
            if st != 0:
                raise RuntimeError(f"fp32 forward failed: {_lib.last_error()}")
        for _ in range(3):
            call()
        steps = max(5, args.steps)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(steps):
            call()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        flop = B * H * T * 4 * N * D
        out[name] = {"shape": {"B": B, "nh": H, "T": T, "N": N, "D": D}, "ms_per_call": round(ms, 4),
                     "tokens_per_s": round(B * T / (ms * 1e-3), 1),
                     "tflops_recurrent_form": round(flop / (ms * 1e-3) / 1e12, 2),
                     "frac_of_f32_peak": round(flop / (ms * 1e-3) / 1e12 / PEAK_F32_TFLOPS, 4)}
        print(f"[f32] {name}: {ms:.3f} ms/call, {B * T / (ms * 1e-3) / 1e6:.3f} M tok/s, "
              f"{flop / (ms * 1e-3) / 1e12:.1f} TFLOP/s (recurrent form)", flush=True)
        del x, v, ctx, rho
    return {"metric": METRIC + " [fp32 path]", "value": out["c1"]["tokens_per_s"], "unit": "tokens/s",
            "steps": max(5, args.steps), "warmup": 3, "ms_per_step": out["c1"]["ms_per_call"],
            "config": {"workload": "fp32 path through the reference surface: C1 in full, and the C2 "
                                   "shape in fp32 under 'c2_shape'", "global_batch": 1, "seq_len": 256,
                                   "parallelism": "single-gpu"},
            "dtype": "f32", **out}


def bench_ceilings(torch):
    """What this device sustains, measured in the same run as the kernels it
    bounds:
      hbm       bdh_calib_hbm on a 2 GiB buffer (C3's rho: 64 x 4 x 8192 rows
                of 1 KiB): a read, a copy, an in-place read-modify-write, and a
                read-modify-write of 5 % / 10 % of the 1 KiB rows picked at
                random (sorted, as a decode step walks each stream's active
                rows; non-temporal stores, as the step's); beside them torch's
                copy_ and in-place add_ on the same buffer.  Bytes moved: read
                = size, copy and RMW = 2 x size, row RMW = 2 x rows x 1 KiB;
      mfma      bdh_calib_mfma: v_mfma_f32_16x16x32_bf16 and
                v_mfma_f32_32x32x16_bf16 on register operands, every CU;
      hipblaslt torch.bmm in bf16 (hipBLASLt) on the C2 gram shape (32 x
                [512 x 8192] . [8192 x 512], the full square) and the C2 state
                shape (32 x [8192 x 512] . [512 x 256])."""
    import numpy as np
    from burn_dragon_amd import _lib
    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731

    def timed(call, reps=10):
        for _ in range(2):
            call()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            call()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps * 1e-3  # seconds

    def calib(kind, buf2, rows, n_rows):
        st = lib.bdh_calib_hbm(kind, p(a), buf2, nbytes, p(rows) if rows is not None else None, n_rows,
                               stream)
        if st != 0:
            raise RuntimeError(_lib.last_error())

    hbm = {"buffer_bytes": None}
    nbytes = 64 * 4 * 8192 * 1024
    hbm["buffer_bytes"] = nbytes
    a = torch.zeros(nbytes // 4, device="cuda", dtype=torch.float32)
    b = torch.empty_like(a)
    sink = torch.zeros(4, device="cuda", dtype=torch.float32)

    def rec(name, sec, moved):
        hbm[name] = {"us": round(sec * 1e6, 2), "bytes": moved, "GBs": round(moved / sec / 1e9, 1)}
        print(f"[ceilings] hbm {name}: {sec * 1e6:.1f} us, {moved / sec / 1e12:.2f} TB/s", flush=True)

    rec("read", timed(lambda: calib(_lib.BDH_CALIB_READ, p(sink), None, 0)), nbytes)
    rec("copy", timed(lambda: calib(_lib.BDH_CALIB_COPY, p(b), None, 0)), 2 * nbytes)
    rec("rmw", timed(lambda: calib(_lib.BDH_CALIB_RMW, None, None, 0)), 2 * nbytes)
    rng = np.random.default_rng(SEED + 9)
    total_rows = nbytes // 1024
    for pct in (5, 10):
        pick = np.sort(rng.choice(total_rows, total_rows * pct // 100, replace=False)).astype(np.int32)
        rows = torch.from_numpy(pick).cuda()
        rec(f"rmw_rows_{pct}pct", timed(lambda: calib(_lib.BDH_CALIB_RMW_ROWS, None, rows, pick.size)),
            2 * pick.size * 1024)
    rec("torch_copy", timed(lambda: b.copy_(a)), 2 * nbytes)
    rec("torch_add_inplace", timed(lambda: a.add_(1.0)), 2 * nbytes)
    del a, b

    mfma = {}
    flop = ctypes.c_double()
    for name, kind, peak in (("v_mfma_f32_16x16x32_bf16", _lib.BDH_CALIB_MFMA_16X16X32_BF16, PEAK_BF16_TFLOPS),
                             ("v_mfma_f32_32x32x16_bf16", _lib.BDH_CALIB_MFMA_32X32X16_BF16, PEAK_BF16_TFLOPS),
                             ("v_mfma_f32_32x32x2_f32", _lib.BDH_CALIB_MFMA_32X32X2_F32, PEAK_F32_TFLOPS)):
        def call():
            if lib.bdh_calib_mfma(kind, 20000, p(sink), ctypes.byref(flop), stream) != 0:
                raise RuntimeError(_lib.last_error())
        sec = timed(call, reps=5)
        mfma[name] = {"us": round(sec * 1e6, 1), "TFLOPs": round(flop.value / sec / 1e12, 1),
                      "frac_of_peak": round(flop.value / sec / 1e12 / peak, 4)}
        print(f"[ceilings] mfma {name}: {flop.value / sec / 1e12:.0f} TFLOP/s", flush=True)

    blas = {}
    g = torch.Generator(device="cuda").manual_seed(SEED + 10)
    q = torch.randn(32, 512, 8192, generator=g, device="cuda").to(torch.bfloat16)
    qt = q.transpose(1, 2).contiguous()  # a contiguous right operand (no transposed view)
    v = torch.randn(32, 512, 256, generator=g, device="cuda").to(torch.bfloat16)
    for name, (x, y) in (("c2_gram", (q, qt)), ("c2_state", (qt, v))):
        fl = 2.0 * x.shape[0] * x.shape[1] * x.shape[2] * y.shape[2]
        sec = timed(lambda: torch.bmm(x, y))
        blas[name] = {"shape": [list(x.shape), list(y.shape)], "us": round(sec * 1e6, 1),
                      "TFLOPs": round(fl / sec / 1e12, 1)}
        print(f"[ceilings] hipblaslt {name}: {sec * 1e6:.1f} us, {fl / sec / 1e12:.0f} TFLOP/s", flush=True)
    del q, qt, v
    return {"hbm": hbm, "mfma": mfma, "hipblaslt": blas,
            "peaks": {"hbm_GBs": PEAK_HBM_GBS, "bf16_TFLOPs": PEAK_BF16_TFLOPS, "f32_TFLOPs": PEAK_F32_TFLOPS}}


# --------------------------------------------------------------------------- #
def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build runs the recurrent-attention path on a "
              "single MI355X (the (batch, head) streams are independent, so N GPUs would each run "
              "B*nh/N of them with no exchange). "
              "Use --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    import burn_dragon_amd as bd
    if not bd.supports_backend():
        print("device is not gfx950", file=sys.stderr)
        sys.exit(2)

    if args.only == "copy":
        bench_copy(torch)
        return
    if args.only in ("rmw", "ceilings"):
        print(json.dumps({"ceilings": bench_ceilings(torch)}), flush=True)
        return
    pre = bench_prefill(torch, args) if args.only in ("all", "prefill") else None
    dec = bench_decode(torch, args) if args.only in ("all", "decode") else None
    lng = bench_long(torch, args) if args.only in ("all", "long") else None
    mdl = bench_model(torch, args) if args.only in ("all", "model") else None
    mdd = bench_model_decode(torch, args) if args.only in ("all", "model-decode") else None
    f32 = bench_f32(torch, args) if args.only in ("all", "f32") else None
    ceil = bench_ceilings(torch) if args.only == "all" else None

    cpu_pre = cpu_dec = None
    if not args.no_cpu_baseline:
        if pre is not None:
            cpu_pre = cpu_baseline_prefill(args.cpu_seconds)
            print(f"[cpu] prefill {cpu_pre['value']} tokens/s on {cpu_pre['cores']} threads",
                  flush=True)
        if dec is not None:
            cpu_dec = cpu_baseline_decode(args.cpu_seconds)
            print(f"[cpu] decode {cpu_dec['value']} tokens/s on {cpu_dec['cores']} threads",
                  flush=True)

    if pre is not None:
        out = {
            "metric": METRIC, "value": round(pre["tokens_per_s"], 1), "unit": "tokens/s",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(pre["ms_per_step"], 4), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
            "config": {"workload": "C2 chunked prefill, one BDH layer: B8 nh4 T512 N8192 D256, "
                                   "chunk 128, bf16 in / fp32 acc, RoPE fused, rho out fp32; the "
                                   "pass replayed from a HIP graph (eager timing under 'eager')",
                       "global_batch": 8, "seq_len": 512, "parallelism": "single-gpu"},
            "roofline": pre["roofline"],
            "cpu_baseline": cpu_pre,
            "eager": pre["eager"],
        }
        if dec is not None:
            dec["cpu_baseline"] = cpu_dec
            out["decode"] = dec
        if lng is not None:
            out["long_prefill"] = lng
        if mdl is not None:
            out["model"] = mdl
        if mdd is not None:
            out["model_decode"] = mdd
        if f32 is not None:
            out["fp32_path"] = f32
        if ceil is not None:
            out["ceilings"] = ceil
    elif dec is None:
        one = next(r for r in (lng, mdl, mdd, f32) if r is not None)
        out = dict(one, n_gpus=1, higher_is_better=True, scaling="weak", vs_baseline=None,
                   data="synthetic")
        out.setdefault("dtype", "bf16")
    else:
        out = {"metric": METRIC, "value": round(dec["value"], 1), "unit": "tokens/s", "n_gpus": 1,
               "steps": dec["steps"], "warmup": dec["warmup"],
               "ms_per_step": round(dec["ms_per_step"], 5), "higher_is_better": True,
               "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
               "config": dec["config"], "roofline": dec["roofline"], "cpu_baseline": cpu_dec}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
