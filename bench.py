"""Benchmark of the fused attention family on one MI355X.

Default workload (the shape BASELINE.json's metric is quoted on):
attention_with_scores, B=1, H=32, M=N=4096, D=128, fp16, causal.  A "step"
is one call of the drop-in entry point over that batch with q/k/v already
resident in HBM.  The line printed is the driver's JSON contract plus
  roofline      dominant kernel vs MI355X peak (HBM for the score-writing
                kernel, fp16 MFMA for the sum-only kernels), from HIP events
                recorded on the stream the kernel runs on;
  cpu_baseline  the CPU oracle (oracle/naive.py, a fp32 restatement of the
                reference's naive attention) timed on a bounded sample of the
                same workload on this host -- a reported baseline only;
  secondary     the softmax column-sum kernel at the same shape against the
                fp16 MFMA peak.

Before the counted warmup steps, every run pre-warms by time: it calls the
step until at least --prewarm-ms (default 150 ms) of wall time has passed,
whatever --warmup says.  From idle, the GPU needs ~25 ms of load to raise its
clocks, and the first calls run up to 30% slower (measured on the MI355X: 302
us per scores call in the first 5 ms, 231 us from ~25 ms on, at the 1400 W
board power limit); a count of warmup calls alone (the driver passes
--warmup 5) would time that ramp, not the kernel.  The reference's harness
warms by time as well (triton.testing.do_bench(warmup=50), benchmark.py:254,
352).  The line reports the pre-warm as "prewarm" and keeps "warmup" as
passed.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0        # MI355X HBM3E, GB/s
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16/bf16 MFMA, TFLOP/s

METRIC = "fused attn TFLOP/s + scores-write GB/s, fp16 H32 S4096 D128 causal"

# name -> (entry point, needs split, roofline bound, flop factor per pair
#          (multiples of B*H*D per admissible pair), side product bytes fn)
WORKLOADS = {
    "scores": ("attention_with_scores", False, "hbm", 4),
    "row_sum": ("attention_with_row_sum", False, "mfma", 4),
    "col_sum": ("attention_with_col_sum", False, "mfma", 4),
    "col_sum_sequential": ("attention_with_col_sum_sequential", False, "mfma", 4),
    "col_softmax": ("attention_with_softmax_col_sum", False, "mfma", 6),
    "cross_qk": ("attention_cross_token_qk_sum", True, "mfma", 4),
    "cross_softmax": ("attention_cross_token_softmax_sum", True, "mfma", None),
    "cross_softmax_buffered": ("attention_cross_token_softmax_sum_buffered", True, "hbm", None),
    # attention()'s forward pass (flash.py:32-169) with inputs that need
    # gradients, as in training: O and L, plus the dropout keep bits the
    # backward reads when dropout is on.
    "attention_fwd": ("attention", False, "mfma", 4),
    # attention()'s backward pass alone (flash.py:172-261), FA2 convention:
    # 2.5x the forward's 4*B*H*D*P.
    "attention_bwd": ("attention", False, "mfma", 10),
    # attention_scores.compute_attention_scores (attention_scores.py:154-223):
    # the unmasked score matrix alone, 2*B*H*M*N*D FLOP.
    "scores_only": ("compute_attention_scores", False, "hbm", 2),
}


def pairs(M: int, N: int, causal: bool, offset: int) -> int:
    """Admissible (query, key) pairs of one head: key j for query i iff
    offset + i >= j when causal."""
    if not causal:
        return M * N
    total = 0
    for i in range(M):
        total += max(0, min(N, offset + i + 1))
    return total


def cross_pairs(M: int, N: int, split: int, causal: bool, offset: int) -> int:
    total = 0
    for i in range(split, M):
        hi = split if not causal else max(0, min(split, offset + i + 1))
        total += hi
    return total


def work(name: str, B, H, Hk, M, N, D, causal, split, elem=2):
    """(algorithmic FLOP, algorithmic HBM bytes) of one call."""
    ep, _, _, fac = WORKLOADS[name]
    off = 0 if name == "cross_qk" else N - M
    P = pairs(M, N, causal, off)
    qkvo = elem * (2 * B * H * M * D + 2 * B * Hk * N * D)
    if name == "scores":
        return 4 * B * H * D * P, qkvo + elem * B * H * M * N
    if name == "scores_only":
        # reads q, k; writes the full score matrix
        return (fac * B * H * M * N * D,
                elem * (B * H * M * D + B * Hk * N * D + B * H * M * N))
    if name in ("row_sum", "attention_fwd"):
        # + the (B, H, M) fp32 row sums / log-normalizer
        return 4 * B * H * D * P, qkvo + 4 * B * H * M
    if name in ("col_sum", "col_sum_sequential", "col_softmax"):
        return fac * B * H * D * P, qkvo + 4 * B * Hk * N
    if name == "attention_bwd":
        # reads q, k, v, o, dO, L; writes dq, dk, dv
        return fac * B * H * D * P, qkvo + elem * (B * H * M * D * 2 + 2 * B * Hk * N * D)
    Px = cross_pairs(M, N, split, causal, off)
    if name == "cross_qk":
        return 4 * B * H * D * P, qkvo + 4 * B * Hk * split
    if name == "cross_softmax":
        return 4 * B * H * D * P + 2 * B * H * D * Px, qkvo + 4 * B * Hk * split
    # buffered: pass 2 reloads the region instead of recomputing its scores.
    # The region leaves pass 1 as fp16 exponents (2 bytes a score) plus one
    # fp32 offset per row and 64-key tile, written once and read once (the
    # reference's raw fp32 scores would be twice the bytes).
    region = B * H * max(M - split, 0) * (2 * split + 4 * ((split + 63) // 64))
    return 4 * B * H * D * P, qkvo + 2 * region + 4 * B * Hk * split


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(name, B, H, Hk, M, N, D, causal, split, dtype, budget_s: float,
                 scale: float = 1.0) -> dict:
    """Times the CPU oracle (oracle/naive.py, the checker) on whole heads of
    the same workload, cycling over the heads until budget_s of work is
    done; the rate counts the heads actually computed."""
    from oracle import inputs, naive

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    q, k, v = inputs.make_qkv(B, H, Hk, M, N, D, dtype=dtype, seed=0, scale=scale)
    ep = WORKLOADS[name][0]
    side = naive.ENTRY_POINT_OUTPUT[ep]
    offset = naive.ENTRY_POINT_OFFSET[ep]
    done = 0
    t0 = time.perf_counter()
    while True:
        h = done % H
        naive.reference_forward(q, k, v, causal=causal, causal_offset=offset, split=split,
                                want=("out", side), heads=[h])
        done += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    elapsed = time.perf_counter() - t0
    flop, _ = work(name, B, H, Hk, M, N, D, causal, split)
    flop_done = flop * done / H
    return {
        "value": round(flop_done / elapsed / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"oracle/naive.py (fp32 restatement of reference_implementations.py) on "
                  f"{done} head-passes ({done / H:.2f}x the {H}-head workload) of {ep} at the "
                  f"bench shape, {elapsed:.1f} s; {cpu_model()}, os.cpu_count()={threads}",
    }


# Measured HBM bytes per launch of the dominant kernel (two rocprofv3 PMC
# passes, FETCH_SIZE and WRITE_SIZE scaled against a copy of known size),
# recorded in a committed summary under profiles/ next to the command that
# produced it.
TRAFFIC_SUMMARIES = {
    ("scores", 1, 32, 32, 4096, 128, "fp16", True): "attn_fwd_scores_f16_b1h32s4096d128_causal.md",
    ("scores_only", 1, 32, 32, 4096, 128, "fp16", True): "scores_only_f16_b1h32s4096d128.md",
}


def measured_traffic(key):
    name = TRAFFIC_SUMMARIES.get(key)
    if name is None:
        return None, None
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("TRAFFIC_BYTES_PER_LAUNCH"):
                    return int(line.split("=")[1]), "profiles/" + name
    except OSError:
        pass
    return None, None


def synthetic_qkv(B, Hq, Hk, M, N, D, dtype, scale, device):
    """q, k, v i.i.d. N(0, 1) * scale, drawn in fp32 from a CPU generator seeded 0
    (q, then k, then v), rounded to `dtype` and moved to `device`."""
    g = torch.Generator("cpu").manual_seed(0)
    out = []
    for shape in ((B, Hq, M, D), (B, Hk, N, D), (B, Hk, N, D)):
        out.append((torch.randn(shape, generator=g, dtype=torch.float32) * scale)
                   .to(dtype).to(device))
    return tuple(out)


def make_call(fas, name, q, k, v, causal, split, dropout_p=0.0):
    if name == "attention_fwd":
        # Each call builds the autograd graph (and, with dropout, the keep
        # bits) and drops it with its output.
        qg, kg, vg = (t.detach().requires_grad_(True) for t in (q, k, v))
        return lambda: fas.attention(qg, kg, vg, causal=causal, dropout_p=dropout_p)
    if name == "attention_bwd":
        # One forward outside the timed calls; each call is one backward pass
        # through the autograd graph (dq, dk, dv).
        qg, kg, vg = (t.detach().requires_grad_(True) for t in (q, k, v))
        o = fas.attention(qg, kg, vg, causal=causal, dropout_p=dropout_p)
        g = torch.Generator(device=q.device).manual_seed(1)
        do = torch.randn(o.shape, generator=g, device=q.device, dtype=o.dtype)
        return lambda: torch.autograd.grad(o, (qg, kg, vg), do, retain_graph=True)
    if name == "scores_only":
        from flash_attn_with_score_amd.attention_scores import compute_attention_scores
        return lambda: compute_attention_scores(q, k)
    fn = getattr(fas, WORKLOADS[name][0])
    if WORKLOADS[name][1]:
        return lambda: fn(q, k, v, split, causal=causal, dropout_p=dropout_p)
    return lambda: fn(q, k, v, causal=causal, dropout_p=dropout_p)


def prewarm(call, min_ms: float) -> dict:
    """Calls `call` in batches of 10 until min_ms of wall time has passed
    (synchronising after each batch), so the clocks have left their ramp
    before anything is timed."""
    calls = 0
    t0 = time.perf_counter()
    while min_ms > 0:
        for _ in range(10):
            call()
        calls += 10
        torch.cuda.synchronize()
        if (time.perf_counter() - t0) * 1e3 >= min_ms:
            break
    return {"ms": round((time.perf_counter() - t0) * 1e3, 1), "calls": calls}


def time_steps(call, steps: int, warmup: int, prewarm_ms: float):
    """Wall time of `steps` calls, bracketed by synchronize, plus the average
    device time per call from HIP events on torch's current stream (the
    stream the entry points launch on).  A time-based pre-warm and then
    `warmup` untimed calls come first."""
    warm = prewarm(call, prewarm_ms)
    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        call()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    dev_ms = start.elapsed_time(end) / steps
    return wall, dev_ms, warm


def time_cold(call, reps: int, flush_bytes: int = 512 << 20) -> float:
    """Average device time of `reps` calls, each timed alone with HIP events
    on torch's current stream right after a read of `flush_bytes` (outside
    the events) that evicts the XCDs' L2 caches and the 256 MB Infinity Cache,
    so every call reads its inputs from HBM.  A read, not a write: a written
    flush leaves up to 256 MB of dirty lines that the timed call would then
    pay to write back."""
    buf = torch.ones(flush_bytes // 4, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()
    events = []
    for _ in range(reps):
        buf.amax()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        call()
        end.record(stream)
        events.append((start, end))
    torch.cuda.synchronize()
    del buf
    return sum(a.elapsed_time(b) for a, b in events) / reps


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--prewarm-ms", type=float, default=150.0,
                    help="wall time of calls before the warmup steps (clock ramp; default 150)")
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="scores")
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--heads", type=int, default=32)
    ap.add_argument("--kv-heads", type=int, default=None)
    ap.add_argument("--seqlen", type=int, default=4096)
    ap.add_argument("--seqlen-q", type=int, default=None,
                    help="query length M (default: --seqlen); keys N = --seqlen")
    ap.add_argument("--head-dim", type=int, default=128)
    ap.add_argument("--split", type=int, default=None)
    ap.add_argument("--dtype", choices=["fp16", "bf16"], default="fp16")
    ap.add_argument("--non-causal", action="store_true")
    ap.add_argument("--dropout", type=float, default=0.0,
                    help="dropout_p of the forward workloads (default 0, as every config)")
    ap.add_argument("--input-scale", type=float, default=1.0,
                    help="q/k/v are N(0,1) times this (BASELINE config 4 uses 0.5)")
    ap.add_argument("--cpu-budget", type=float, default=12.0,
                    help="seconds of CPU-oracle work for cpu_baseline (0 disables)")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run one 256 MiB device-to-device copy first (a kernel of known HBM "
                         "traffic for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the path shards by (batch, KV-head group) with no communication, so N GPUs "
              "run N independent copies -- no multi-GPU figure is produced.", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 1

    import flash_attn_with_score_amd as fas

    dtype = torch.float16 if args.dtype == "fp16" else torch.bfloat16
    B, H, N, D = args.batch, args.heads, args.seqlen, args.head_dim
    M = args.seqlen_q or N
    Hk = args.kv_heads or H
    causal = not args.non_causal
    split = args.split
    if WORKLOADS[args.workload][1] and split is None:
        split = (3 * N) // 4
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.calibrate_copy:
        src = torch.ones(128 << 20, dtype=torch.float16, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    q, k, v = synthetic_qkv(B, H, Hk, M, N, D, dtype, args.input_scale, dev)
    if args.dropout and args.workload == "scores_only":
        print(f"--dropout does not apply to {args.workload}", file=sys.stderr)
        return 2
    call = make_call(fas, args.workload, q, k, v, causal, split, args.dropout)
    wall, dev_ms, warm = time_steps(call, args.steps, args.warmup, args.prewarm_ms)
    flop, nbytes = work(args.workload, B, H, Hk, M, N, D, causal, split)
    ms = wall * 1e3 / args.steps
    tflops = flop / (ms * 1e-3) / 1e12
    bound = WORKLOADS[args.workload][2]
    if bound == "hbm":
        achieved = nbytes / (dev_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4)}
    else:
        achieved = flop / (dev_ms * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / MFMA_F16_PEAK_TFLOPS, 4)}
    traffic, source = measured_traffic((args.workload, B, H, Hk, M, D, args.dtype, causal))
    roof["traffic"] = traffic
    if traffic is not None:
        roof["traffic_source"] = source
    roof["kernel_ms"] = round(dev_ms, 4)
    if bound == "hbm":
        # The same calls with the caches evicted before each one.
        cold_ms = time_cold(call, 20)
        roof["kernel_ms_cold"] = round(cold_ms, 4)
        roof["frac_cold"] = round(nbytes / (cold_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)
    roof["algorithmic_bytes"] = nbytes
    roof["algorithmic_flop"] = flop

    line = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "prewarm": warm,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic: q/k/v i.i.d. N(0,1)"
                + (f" x {args.input_scale:g}" if args.input_scale != 1.0 else "")
                + " from a seeded CPU generator",
        "config": {"workload": f"{WORKLOADS[args.workload][0]} B{B} H{H}/{Hk} "
                               + (f"S{M}" if M == N else f"M{M} N{N}")
                               + f" D{D} {args.dtype} {'causal' if causal else 'full'}"
                               + (f" split{split}" if split else ""),
                   "batch": B, "heads_q": H, "heads_k": Hk, "seqlen": M, "seqlen_k": N,
                   "head_dim": D,
                   "causal": causal, "split": split, "dropout_p": args.dropout,
                   "parallelism": "none (1 GPU)"},
        "flop_convention": "4*B*H*D*(admissible pairs) (causal work); "
                           "reference convention 4*B*H*M*N*D in tflops_ref_convention",
        "tflops_ref_convention": round(4 * B * H * M * N * D / (ms * 1e-3) / 1e12, 2),
        "hbm_GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
    }
    if args.workload == "scores":
        line["scores_write_GBps"] = round(2 * B * H * M * N / (ms * 1e-3) / 1e9, 1)
    line["roofline"] = roof

    if not args.no_secondary and args.workload == "scores":
        call2 = make_call(fas, "col_softmax", q, k, v, causal, None)
        _, dev2, _ = time_steps(call2, max(5, args.steps // 2), max(2, args.warmup // 2),
                                args.prewarm_ms)
        flop2, _ = work("col_softmax", B, H, Hk, M, N, D, causal, None)
        a2 = flop2 / (dev2 * 1e-3) / 1e12
        line["secondary"] = {"workload": f"attention_with_softmax_col_sum B{B} H{H} S{M} D{D} "
                                         f"{args.dtype} {'causal' if causal else 'full'}",
                             "kernel_ms": round(dev2, 4), "achieved": round(a2, 1),
                             "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(a2 / MFMA_F16_PEAK_TFLOPS, 4)}

    del q, k, v
    torch.cuda.synchronize()
    if args.cpu_budget > 0 and args.workload not in ("attention_fwd", "attention_bwd", "scores_only"):
        line["cpu_baseline"] = cpu_baseline(args.workload, B, H, Hk, M, N, D, causal, split,
                                            dtype, args.cpu_budget, args.input_scale)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
