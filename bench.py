#!/usr/bin/env python3
"""Benchmark of the attention block: fwd+bwd tokens/s and peak HBM on one GPU.

Workload: the 50M-pretrain block shape B=64, T=4096, C=512, H=8, N=64, bf16
(262,144 tokens per step), synthetic seeded inputs resident in HBM before
the timed region. A step is one forward and one backward of
FusedAttentionFunction over the whole batch (input and all five weight
gradients; the rotary tables are buffers, as in a YaRN module).

Printed on stdout: ONE JSON line with the metric, the per-kernel roofline of
the dominant kernel (timed live with HIP events on its launch stream over the
timed region, the only launches the events bracket there; every kernel's
average comes from an equal pass just before, with events around each
launch), peak HBM, and the CPU baseline (the fp32 oracle on a bounded
batch slice on the host cores). Progress goes to stderr.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-eager] [--no-cpu-baseline] [--no-box-reference] [--table-grad]
    python bench.py --workload 2|3       # the same line for another fwd+bwd workload
    python bench.py --workload 4         # forward-only (prefill) workload: fwd tokens/s, no CPU leg
    python bench.py --workload W --varlen  # B packed sequences of seeded lengths in [T/4, T], fwd+bwd
    python bench.py --workload W --decode [--context L]
                                         # KV-cache decode steps at context L (default T - 1)
    python bench.py --copy-calibration   # a plain 256 MiB device copy, for HBM counter scaling
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

METRIC = "fwd+bwd tokens/s & peak mem, attn block bf16 B64 T4096 C512 H8 N64"


def metric_of(w) -> str:
    """The metric string of a workload (the headline one, B64 T4096 C512 H8 N64, for workload 1)."""
    kind = "fwd+bwd" if w.backward else "fwd (prefill, no grad)"
    return f"{kind} tokens/s & peak mem, attn block bf16 B{w.B} T{w.T} C{w.C} H{w.H} N{w.N}"
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0
ROOT = Path(__file__).resolve().parent


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def kernel_work(w):
    """Algorithmic flops and bytes per launch of each kernel.
    Attention pairs are counted exactly (causal T(T+1)/2); a product that a
    kernel recomputes (S in both backward kernels, dP in the dQ kernel) is
    not algorithmic work and is not counted."""
    B, T, C, H, N = w.B, w.T, w.C, w.H, w.N
    M, HN = B * T, H * N
    pair = 2.0 * B * H * N * T * (T + 1) / 2  # flops of one causal (T x T x N) product
    return {
        "qkvg_proj": dict(flops=2.0 * M * C * 4 * HN, bytes=2.0 * M * C + 2.0 * 4 * M * HN),
        "attn_fwd": dict(flops=2 * pair, bytes=2.0 * 4 * M * HN),
        "gate_oproj": dict(flops=2.0 * M * HN * C, bytes=2.0 * 2 * M * HN + 2.0 * M * C),
        # reads dy, O, sigmoid(a_g); writes dO, da_g and z = O * sigmoid(a_g)
        "dz_gate_bwd": dict(flops=2.0 * M * C * HN, bytes=2.0 * M * C + 2.0 * 5 * M * HN),
        "attn_bwd_dq": dict(flops=1 * pair, bytes=2.0 * 5 * M * HN),
        "attn_bwd_dkdv": dict(flops=3 * pair, bytes=2.0 * 6 * M * HN),
        # reads da (4 parts), x, dy and z
        "dw_partial": dict(flops=2.0 * M * (4 * HN * C + C * HN), bytes=2.0 * M * (4 * HN + C + C + HN)),
        "dx": dict(flops=2.0 * M * 4 * HN * C, bytes=2.0 * M * (4 * HN + 2 * C)),
    }


def cpu_model() -> str:
    """The host CPU as /proc/cpuinfo names it: the full "model name" string of
    the first processor entry, with its vendor, family, model and stepping
    numbers (a virtual machine may report a shortened model name) and the
    logical processors listed."""
    try:
        fields, nproc = {}, 0
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            key, _, val = line.partition(":")
            key = key.strip()
            if key == "processor":
                nproc += 1
            if nproc == 1 and key in ("model name", "vendor_id", "cpu family", "model", "stepping"):
                fields[key] = val.strip()
        name = fields.get("model name", "unknown")
        ids = ", ".join(f"{k} {fields[k]}" for k in ("vendor_id", "cpu family", "model", "stepping") if k in fields)
        return f"{name} ({ids}; {nproc} logical processors in /proc/cpuinfo)"
    except OSError:
        return "unknown"


def cpu_baseline(w, seconds: float):
    """The fp32 oracle (eager block, CPU) on a batch slice of the workload."""
    import torch

    from memory_efficient_attn_layer_amd.synthetic import make_inputs
    from oracle import block as ob

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))
    threads = max(1, min(threads, len(os.sched_getaffinity(0))))
    torch.set_num_threads(threads)
    inp = make_inputs(w, B=1, dtype=torch.float32)
    ob.block_grads(inp, w.H, w.N, dtype=torch.float32)  # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < seconds and len(times) < 20):
        t0 = time.perf_counter()
        ob.block_grads(inp, w.H, w.N, dtype=torch.float32)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > 3 * seconds:
            break
    med = statistics.median(times)
    per_seq = 3.4 * w.H * w.T * w.T * 4
    return {
        "value": w.T / med,
        "unit": "tokens/s",
        "cores": threads,
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": f"fp32 oracle fwd+bwd (oracle/block.py) on 1 of {w.B} sequences (T={w.T}, C={w.C}, "
                  f"H={w.H}, N={w.N}); 1 warm-up + {len(times)} timed iterations, median {med:.2f} s. "
                  f"One sequence, because the oracle's math-path SDPA keeps fp32 (H, T, T) scores and "
                  f"probabilities per sequence for the backward (about 3.4 H T^2 4 bytes = {per_seq / 1e9:.1f} GB "
                  f"of host memory per sequence, measured 1.8 GB at T=4096, H=8; {w.B * per_seq / 1e9:.0f} GB "
                  f"for all {w.B}); sequences are independent, so the cost is linear in B and value = T / median "
                  f"is the per-token rate of the whole batch",
    }


def eager_block(x, wq, wk, wv, wg, wo, f1, f2, H, N):
    """The reference's eager path on the GPU (README.md:42-64): checkpointed
    projections + SDPA flash + gate + o_proj, in bf16."""
    import torch
    import torch.nn.functional as F
    from torch.utils.checkpoint import checkpoint

    from memory_efficient_attn_layer_amd.yarn import swap_even_odd

    B, T, C = x.shape
    fs1, fs2 = f1[:T, None, :], f2[:T, None, :]

    def forward1(x):
        x = F.rms_norm(x, (C,), eps=1e-6)
        q = F.linear(x, wq).view(B, T, H, N)
        k = F.linear(x, wk).view(B, T, H, N)
        v = F.linear(x, wv).view(B, T, H, N)
        g = F.linear(x, wg)
        q = F.rms_norm(q, (N,), eps=1e-6)
        k = F.rms_norm(k, (N,), eps=1e-6)
        q = q * fs1 + swap_even_odd(q) * fs2
        k = k * fs1 + swap_even_odd(k) * fs2
        return q, k, v, g

    q, k, v, g = checkpoint(forward1, x, use_reentrant=False)
    with torch.nn.attention.sdpa_kernel(torch.nn.attention.SDPBackend.FLASH_ATTENTION):
        o = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                           is_causal=True).transpose(1, 2).contiguous().view(B, T, H * N)
    return F.linear(o * torch.sigmoid(g), wo)


def measure(step, steps, warmup, sync):
    for _ in range(warmup):
        step()
    sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    sync()
    return (time.perf_counter() - t0) / steps


def measure_and_profile(step, steps, sync, candidates):
    """Per-kernel averages and the timed steps.

    First `steps` steps run with the library's HIP events (recorded on the
    launch stream) around every kernel; they give each kernel's launch count
    and total time and name the dominant kernel, the one of `candidates` with
    the largest total. Then the timed region: `steps` more steps with events
    around the dominant kernel's launches only, whose figures replace that
    kernel's entry. Every event pair adds about 8 us of queue time to a step
    (1.9% of the B64 T4096 step with all of them), so the timed steps carry
    just the pairs the roofline needs. Returns (seconds per timed step,
    {kernel: (launches, total ms)}, dominant kernel)."""
    from memory_efficient_attn_layer_amd import _lib

    _lib.profile_select(None)
    _lib.profile_enable(True)
    measure(step, steps, 0, sync)
    _lib.profile_enable(False)
    prof = _lib.profile_read()
    dom = max((k for k in prof if k in candidates), key=lambda k: prof[k][1])
    _lib.profile_select(dom)
    _lib.profile_enable(True)
    sec = measure(step, steps, 0, sync)
    _lib.profile_enable(False)
    prof[dom] = _lib.profile_read()[dom]
    _lib.profile_select(None)
    return sec, prof, dom


def peak_of(step, sync):
    import torch

    sync()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    step()
    sync()
    return torch.cuda.max_memory_allocated() - base


def box_reference():
    """Speed of this GPU on two vendor operations, for comparing runs made on
    different machines: a bf16 matrix product of 8192^3 (torch.matmul of two
    contiguous 2-D tensors) in TFLOP/s and a 1 GiB device-to-device copy in
    GB/s (bytes read plus written). Measured outside the timed region."""
    import torch

    def timed(fn, reps):
        for _ in range(3):
            fn()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        b.synchronize()
        return a.elapsed_time(b) * 1e-3 / reps

    n = 8192
    g = torch.Generator(device="cuda").manual_seed(7)
    x = torch.randn(n, n, device="cuda", dtype=torch.bfloat16, generator=g)
    y = torch.randn(n, n, device="cuda", dtype=torch.bfloat16, generator=g)
    gemm = 2 * n**3 / timed(lambda: torch.matmul(x, y), 10) / 1e12
    del x, y
    src = torch.empty(2**30, device="cuda", dtype=torch.uint8)
    dst = torch.empty_like(src)
    copy = 2 * 2**30 / timed(lambda: dst.copy_(src), 10) / 1e9
    del src, dst
    torch.cuda.empty_cache()
    return {"gemm_bf16_tflops": round(gemm, 1), "copy_gbs": round(copy, 1)}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", type=int, default=1, help="workload id (1 = the headline shape, B64 T4096 C512 H8 N64)")
    ap.add_argument("--no-eager", action="store_true",
                    help="skip the eager checkpoint+SDPA comparator (timed and peak HBM on the same GPU)")
    ap.add_argument("--table-grad", action="store_true",
                    help="also differentiate the (bf16) rotary tables (dF1 / dF2, as the reference always does)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-box-reference", action="store_true",
                    help="skip the vendor GEMM / copy speed reference (keeps kernel traces to this library)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--varlen", action="store_true",
                    help="pack B sequences of seeded random lengths in [T/4, T] (fwd+bwd, packed-sequence path)")
    ap.add_argument("--decode", action="store_true",
                    help="time KV-cache decode steps (one token per sequence) instead of fwd+bwd")
    ap.add_argument("--context", type=int, default=None, help="decode: cached tokens per sequence (default T - 1)")
    ap.add_argument("--graph", action="store_true", help="decode: also time the step replayed from a captured graph")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain device copy of 256 MiB five times (reference for HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported; this block runs on one GPU only "
              "(no collective or sharded path is built). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_calibration:
        n = 256 << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "launches": 5}), flush=True)
        return

    from memory_efficient_attn_layer_amd import _lib
    from memory_efficient_attn_layer_amd.attention import FusedAttentionFunction
    from memory_efficient_attn_layer_amd.synthetic import WORKLOADS, make_inputs

    w = WORKLOADS[args.workload]
    if args.decode:
        decode_bench(args, w)
        return
    if args.varlen:
        varlen_bench(args, w)
        return
    if not w.backward:
        forward_bench(args, w)
        return
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    log(f"workload {w.name}; generating inputs")
    inp = make_inputs(w, device=dev)
    x = inp["x"].requires_grad_(True)
    ws = [inp[n].requires_grad_(True) for n in ("wq", "wk", "wv", "wg", "wo")]
    f1, f2, dy = inp["f1"], inp["f2"], inp["dy"]
    wrt = [x, *ws]
    if args.table_grad:
        # Trainable tables, differentiated like every other input. They stay
        # bf16, as the reference's tables are, so the step differs from the
        # plain one only by the table gradients (dF1 / dF2).
        f1 = f1.detach().clone().requires_grad_(True)
        f2 = f2.detach().clone().requires_grad_(True)
        wrt += [f1, f2]
    H, N = w.H, w.N
    sync = torch.cuda.synchronize

    def step():
        y = FusedAttentionFunction.apply(x, *ws, f1, f2, H, N, 1e-6)
        return torch.autograd.grad(y, wrt, dy)

    log("warm-up")
    for _ in range(max(1, args.warmup)):
        step()
    sync()
    peak = peak_of(step, sync)
    log(f"peak HBM over one step: {peak / 2**20:.1f} MiB")

    work = kernel_work(w)
    sec, prof, _ = measure_and_profile(step, args.steps, sync, work)
    ms = sec * 1e3
    tokens = w.B * w.T
    log(f"{ms:.3f} ms/step, {tokens / sec / 1e6:.2f} M tokens/s")

    kernels = {}
    for name, (cnt, tot) in sorted(prof.items(), key=lambda kv: -kv[1][1]):
        avg = tot / cnt
        ent = {"launches_per_step": cnt / args.steps, "avg_ms": round(avg, 4), "share": round(tot / (ms * args.steps), 4)}
        if name in work:
            ent["tflops"] = round(work[name]["flops"] / (avg * 1e-3) / 1e12, 2)
            ent["gbs"] = round(work[name]["bytes"] / (avg * 1e-3) / 1e9, 1)
        kernels[name] = ent
        log(f"  {name:15s} {avg:8.4f} ms x{cnt / args.steps:.0f}  {ent.get('tflops', '-')} TFLOP/s")
    dom = max((k for k in prof if k in work), key=lambda k: prof[k][1])
    avg_s = prof[dom][1] / prof[dom][0] * 1e-3
    achieved = work[dom]["flops"] / avg_s / 1e12
    # HBM bytes per launch from the committed FETCH_SIZE / WRITE_SIZE runs,
    # which cover the headline workload (B64 T4096 C512 H8 N64) only.
    traffic = None
    tfile = ROOT / "profiles" / "traffic.json"
    if w.wid == 1 and tfile.exists():
        try:
            traffic = json.loads(tfile.read_text()).get(dom)
        except (ValueError, OSError):
            traffic = None
    roofline = {"kernel": dom, "bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": traffic}
    # The three attention kernels together: algorithmic flops (forward 2, backward
    # 4 causal products) and the products the hardware runs (the backward
    # recomputes S twice and dP once more).
    attn = ("attn_fwd", "attn_bwd_dq", "attn_bwd_dkdv")
    if all(k in prof for k in attn):
        pair = work["attn_bwd_dq"]["flops"]
        t_attn = sum(prof[k][1] / prof[k][0] for k in attn) * 1e-3
        attention = {"ms": round(t_attn * 1e3, 4), "alg_tflops": round(6 * pair / t_attn / 1e12, 2),
                     "alg_frac": round(6 * pair / t_attn / 1e12 / PEAK_BF16_TFLOPS, 4),
                     "hw_tflops": round(9 * pair / t_attn / 1e12, 2),
                     "hw_frac": round(9 * pair / t_attn / 1e12 / PEAK_BF16_TFLOPS, 4)}
    else:
        attention = None

    eager = None
    if not args.no_eager:
        log("eager SDPA comparator")
        try:
            def estep():
                y = eager_block(x, *ws, f1, f2, H, N)
                return torch.autograd.grad(y, wrt, dy)

            epeak = peak_of(estep, sync)
            esec = measure(estep, max(3, args.steps // 4), 2, sync)
            eager = {"tokens_per_s": round(tokens / esec, 1), "ms_per_step": round(esec * 1e3, 3),
                     "peak_hbm_bytes": int(epeak)}
            log(f"eager: {esec * 1e3:.3f} ms/step, peak {epeak / 2**20:.1f} MiB")
        except Exception as e:  # noqa: BLE001 - report, do not fail the benchmark
            eager = {"error": f"{type(e).__name__}: {e}"[:300]}

    box = None if args.no_box_reference else box_reference()
    if box:
        log(f"box reference: bf16 GEMM {box['gemm_bf16_tflops']} TFLOP/s, copy {box['copy_gbs']} GB/s")

    cpu = None
    if not args.no_cpu_baseline:
        log("CPU baseline (fp32 oracle)")
        cpu = cpu_baseline(w, args.cpu_seconds)
        log(f"cpu: {cpu['value']:.1f} tokens/s on {cpu['cores']} cores")

    out = {
        "metric": metric_of(w),
        "value": round(tokens / sec, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": w.name, "B": w.B, "T": w.T, "C": w.C, "H": H, "N": N,
                   "tokens_per_step": tokens, "table_grad": bool(args.table_grad), "parallelism": "single-gpu"},
        "peak_hbm": {"fused_bytes": int(peak), "eager_sdpa": eager,
                     "fused_below_eager": None if not eager or "peak_hbm_bytes" not in eager
                     else bool(peak < eager["peak_hbm_bytes"])},
        "block_tflops": round(3 * w.flops_fwd() / sec / 1e12, 2),
        "roofline": roofline,
        "attention": attention,
        "kernels": kernels,
        "box_reference": box,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def roofline_of(prof, work):
    """Roofline entry of the kernel with the largest total time."""
    dom = max((k for k in prof if k in work), key=lambda k: prof[k][1])
    avg_s = prof[dom][1] / prof[dom][0] * 1e-3
    achieved = work[dom]["flops"] / avg_s / 1e12
    return {"kernel": dom, "bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": None}


def forward_bench(args, w):
    """Forward-only (prefill) workload: the inference forward under no_grad
    (no saved O / lse), timed like the training step. The fp32 CPU oracle
    cannot run a sequence of this length in bounded time, so there is no CPU
    leg."""
    import torch

    from memory_efficient_attn_layer_amd import _lib
    from memory_efficient_attn_layer_amd.attention import FusedAttentionFunction
    from memory_efficient_attn_layer_amd.synthetic import make_inputs

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    log(f"workload {w.name} (forward only); generating inputs")
    inp = make_inputs(w, device=dev)
    args_in = [inp[n] for n in ("x", "wq", "wk", "wv", "wg", "wo", "f1", "f2")]
    sync = torch.cuda.synchronize

    def step():
        with torch.no_grad():
            return FusedAttentionFunction.apply(*args_in, w.H, w.N, 1e-6)

    log("warm-up")
    for _ in range(max(1, args.warmup)):
        step()
    sync()
    peak = peak_of(step, sync)
    work = kernel_work(w)
    sec, prof, _ = measure_and_profile(step, args.steps, sync, work)
    tokens = w.B * w.T
    log(f"{sec * 1e3:.3f} ms/step, {tokens / sec / 1e6:.3f} M tokens/s, peak {peak / 2**20:.1f} MiB")
    kernels = {}
    for name, (cnt, tot) in sorted(prof.items(), key=lambda kv: -kv[1][1]):
        avg = tot / cnt
        ent = {"launches_per_step": cnt / args.steps, "avg_ms": round(avg, 4), "share": round(tot / (sec * 1e3 * args.steps), 4)}
        if name in work:
            ent["tflops"] = round(work[name]["flops"] / (avg * 1e-3) / 1e12, 2)
        kernels[name] = ent
        log(f"  {name:15s} {avg:8.4f} ms x{cnt / args.steps:.0f}  {ent.get('tflops', '-')} TFLOP/s")
    out = {
        "metric": metric_of(w),
        "value": round(tokens / sec, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": w.name, "B": w.B, "T": w.T, "C": w.C, "H": w.H, "N": w.N,
                   "tokens_per_step": tokens, "parallelism": "single-gpu"},
        "peak_hbm": {"fused_bytes": int(peak)},
        "block_tflops": round(w.flops_fwd() / sec / 1e12, 2),
        "roofline": roofline_of(prof, work),
        "kernels": kernels,
        "box_reference": None if args.no_box_reference else box_reference(),
        "cpu_baseline": None,
    }
    print(json.dumps(out), flush=True)


def varlen_bench(args, w):
    """Packed sequences: the workload's B sequences get seeded random lengths
    in [T/4, T] and run back to back through the packed-sequence entry points
    (one forward and one backward per step). Algorithmic attention flops are
    summed per sequence."""
    import torch

    from memory_efficient_attn_layer_amd import _lib
    from memory_efficient_attn_layer_amd.attention import FusedAttentionVarlenFunction
    from memory_efficient_attn_layer_amd.synthetic import make_inputs

    g = torch.Generator().manual_seed(4242)
    lens = torch.randint(w.T // 4, w.T + 1, (w.B,), generator=g).tolist()
    total = sum(lens)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    log(f"workload {w.name}: {w.B} packed sequences, {total} tokens (lengths {min(lens)}..{max(lens)})")
    inp = make_inputs(w, device=dev)
    x = inp["x"].reshape(-1, w.C)[:total].contiguous().requires_grad_(True)
    dy = inp["dy"].reshape(-1, w.C)[:total].contiguous()
    ws = [inp[n].requires_grad_(True) for n in ("wq", "wk", "wv", "wg", "wo")]
    f1, f2 = inp["f1"], inp["f2"]
    del inp
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32, device=dev)
    H, N, L = w.H, w.N, max(lens)
    sync = torch.cuda.synchronize

    def step():
        y = FusedAttentionVarlenFunction.apply(x, *ws, f1, f2, cu, L, H, N, 1e-6)
        return torch.autograd.grad(y, [x, *ws], dy)

    for _ in range(max(1, args.warmup)):
        step()
    sync()
    peak = peak_of(step, sync)
    pair = sum(2.0 * H * N * n * (n + 1) / 2 for n in lens)
    M, HN, C = total, H * N, w.C
    work = kernel_work(w)
    for k in ("qkvg_proj", "gate_oproj", "dz_gate_bwd", "dw_partial", "dx"):
        work[k] = dict(work[k], flops=work[k]["flops"] * M / (w.B * w.T))
    work["attn_fwd"] = dict(work["attn_fwd"], flops=2 * pair)
    work["attn_bwd_dq"] = dict(work["attn_bwd_dq"], flops=pair)
    work["attn_bwd_dkdv"] = dict(work["attn_bwd_dkdv"], flops=3 * pair)
    sec, prof, _ = measure_and_profile(step, args.steps, sync, work)
    kernels = {}
    for name, (cnt, tot) in sorted(prof.items(), key=lambda kv: -kv[1][1]):
        avg = tot / cnt
        ent = {"launches_per_step": cnt / args.steps, "avg_ms": round(avg, 4), "share": round(tot / (sec * 1e3 * args.steps), 4)}
        if name in work:
            ent["tflops"] = round(work[name]["flops"] / (avg * 1e-3) / 1e12, 2)
        kernels[name] = ent
        log(f"  {name:15s} {avg:8.4f} ms x{cnt / args.steps:.0f}  {ent.get('tflops', '-')} TFLOP/s")
    flops = 3 * (2.0 * M * C * 4 * HN + 2 * pair + 2.0 * M * HN * C)
    log(f"{sec * 1e3:.3f} ms/step, {total / sec / 1e6:.2f} M tokens/s")
    out = {
        "metric": f"fwd+bwd tokens/s, {w.B} packed sequences of lengths in [{w.T // 4}, {w.T}], attn block bf16 "
                  f"C{C} H{H} N{N}",
        "value": round(total / sec, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": w.name, "sequences": w.B, "tokens_per_step": total, "max_len": L, "C": C, "H": H,
                   "N": N, "parallelism": "single-gpu"},
        "peak_hbm": {"fused_bytes": int(peak)},
        "block_tflops": round(flops / sec / 1e12, 2),
        "roofline": roofline_of(prof, work),
        "kernels": kernels,
        "box_reference": None if args.no_box_reference else box_reference(),
        "cpu_baseline": None,
    }
    print(json.dumps(out), flush=True)


def decode_bench(args, w):
    """KV-cache decode: a prompt of L tokens per sequence is prefilled, then
    every timed step decodes one token per sequence at position L (the same
    position each step, so every step reads the same L + 1 cache rows). The
    step is bound by HBM: the roofline is the decode attention's cache bytes
    per launch over its live average duration, against 8 TB/s."""
    import torch

    from memory_efficient_attn_layer_amd import _lib
    from memory_efficient_attn_layer_amd.decode import DecodeGraph, KVCache, decode_step, prefill
    from memory_efficient_attn_layer_amd.synthetic import make_inputs

    L = w.T - 1 if args.context is None else int(args.context)
    if not 0 <= L < w.T:
        raise SystemExit(f"--context must be in [0, {w.T - 1}] for workload {w.wid}")
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    log(f"workload {w.name}: decode at context {L}; generating inputs")
    inp = make_inputs(w, device=dev)
    H, N, B, C = w.H, w.N, w.B, w.C
    wts = [inp[n] for n in ("wq", "wk", "wv", "wg", "wo")]
    f1, f2 = inp["f1"].float(), inp["f2"].float()
    cache = KVCache.empty(B, H, N, w.T, dev)
    if L > 0:
        prefill(inp["x"][:, :L], *wts, f1, f2, H, N, cache)
    xt = inp["x"][:, min(L, w.T - 1)].contiguous()
    pos = torch.full((B,), L, dtype=torch.int32, device=dev)
    del inp
    sync = torch.cuda.synchronize

    def step():
        return decode_step(xt, *wts, f1, f2, H, N, pos, cache)

    for _ in range(max(1, args.warmup)):
        step()
    sync()
    peak = peak_of(step, sync)
    steps = max(args.steps, 50)
    sec, prof, _ = measure_and_profile(step, steps, sync, {"attn_decode"})
    HN = H * N
    kv_bytes = 2.0 * B * H * (L + 1) * N * 2
    w_bytes = 2.0 * 5 * HN * C
    kernels = {}
    for name, (cnt, tot) in sorted(prof.items(), key=lambda kv: -kv[1][1]):
        kernels[name] = {"launches_per_step": cnt / steps, "avg_ms": round(tot / cnt, 5),
                         "share": round(tot / (sec * 1e3 * steps), 4)}
        log(f"  {name:20s} {tot / cnt * 1e3:9.2f} us")
    dec_ms = prof["attn_decode"][1] / prof["attn_decode"][0]
    achieved = kv_bytes / (dec_ms * 1e-3) / 1e9
    log(f"{sec * 1e6:.1f} us/step, {B / sec:.0f} tokens/s; cache read {achieved:.0f} GB/s")
    eager_sec = sec
    if args.graph:
        graph = DecodeGraph(*wts, f1, f2, H, N, cache)
        sec = measure(lambda: graph.step(xt, pos), steps, 5, sync)
        log(f"graph replay: {sec * 1e6:.1f} us/step, {B / sec:.0f} tokens/s")
    out = {
        "metric": f"decode tokens/s (one token per sequence per step) at context {L}, attn block bf16 "
                  f"B{B} C{C} H{H} N{N}",
        "value": round(B / sec, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": w.name, "B": B, "context": L, "C": C, "H": H, "N": N,
                   "cache_bytes_read_per_step": int(kv_bytes), "weight_bytes_per_step": int(w_bytes),
                   "parallelism": "single-gpu"},
        "step_hbm_gbs": round((kv_bytes + w_bytes) / sec / 1e9, 1),
        "graph": bool(args.graph),
        "eager_ms_per_step": round(eager_sec * 1e3, 5),
        "peak_hbm": {"step_bytes": int(peak)},
        "roofline": {"kernel": "attn_decode", "bound": "hbm", "achieved": round(achieved, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": None},
        "kernels": kernels,
        "box_reference": None if args.no_box_reference else box_reference(),
        "cpu_baseline": None,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
