"""Benchmark of the Per-Slot EMA hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload attention|scan]

Default workload (configuration 2 of the task): one flash-EMA gated attention layer,
forward + backward, B=56, T=512, d_model=512, 8 heads x 64, N=64 EMA rates, V=50257,
Zipf(1.1) tokens, c_base from a 4096-token warm-up per sequence, weights N(0, 0.02),
dO N(0, 1) (synthetic, seeded).  One step = key-side chunk states (mb_ema_boundary_states)
+ forward (mb_flash_ema_fwd) + backward (mb_flash_ema_bwd), all inputs resident in HBM.

Prints one JSON line.  `roofline` is for the dominant kernel (the backward): algorithmic
flops per launch, sum_b L*K_b*(4*N*D + 10*D) (gate recompute, dW_pe and the five
per-element products; only valid (t, k) pairs count), over its mean launch time measured
with HIP events on the launch stream, against the dense bf16 MFMA peak of 2516.6 TFLOP/s.
`cpu_baseline` times the CPU restatement of the reference algorithm (the oracle, a port
of the reference's PyTorch path) on a bounded slice of the same workload on this host.

`--workload scan` measures the EMA query scan of configuration 3 instead (B=56, T=2048,
N=128, c_base from an 8192-token warm-up) in GB/s of algorithmic traffic.
`--workload copy` runs a plain 1 GiB device-to-device copy: the reference dispatch that
scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters to bytes.
"""
import argparse
import json
import math
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2516.6
PEAK_HBM_GBS = 8000.0

# HBM bytes per dispatch of the dominant kernels, from the rocprofv3 FETCH_SIZE and
# WRITE_SIZE passes scaled by a 1 GiB copy (profiles/flash_ema_cfg2.md); re-measured
# whenever the kernel changes.
TRAFFIC_BYTES = {
    "flash_ema_bwd_kernel": 7522.8e6,
}


def _events():
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def attention_case(seed=0):
    from mathbrain_amd.synthetic import make_batch
    B, L, H, hd, N, V = 56, 512, 8, 64, 64, 50257
    d = make_batch(B, L, V, N, 4096, seed=seed)
    dev = torch.device("cuda", torch.cuda.current_device())
    g = torch.Generator().manual_seed(seed + 1)
    K = d["unique"].shape[1]
    D = H * hd
    c = dict(B=B, L=L, H=H, hd=hd, N=N, V=V, K=K, D=D, counts=d["counts"])
    c["x"] = d["x"].to(dev)
    c["unique"] = d["unique"].to(dev)
    c["c_base"] = d["c_base"].to(dev)
    c["rhos"] = d["rhos"].to(dev)
    c["Q"] = (torch.randn(B, H, L, hd, generator=g) * 0.02).to(dev)
    c["E_k"] = (torch.randn(B, K, D, generator=g) * 0.02).to(dev)
    c["E_v"] = (torch.randn(B, K, D, generator=g) * 0.02).to(dev)
    c["W"] = (torch.randn(N, D, generator=g) * 0.02).to(dev)
    c["dO"] = torch.randn(B, H, L, hd, generator=g).to(dev)
    c["cpu"] = d
    return c


def attention_step(c, timers=None):
    from mathbrain_amd.flash_ema import flash_ema_backward, flash_ema_forward, precompute_boundaries
    Cb = precompute_boundaries(c["x"], c["unique"], c["rhos"], 64, c["c_base"])
    if timers is not None:
        timers["fwd"][0].record()
    O, LSE, *_ = flash_ema_forward(c["Q"], c["x"], c["E_k"], c["E_v"], c["W"], c["rhos"], c["V"],
                                   c["unique"], c["K"], Cb)
    if timers is not None:
        timers["fwd"][1].record()
        timers["bwd"][0].record()
    grads = flash_ema_backward(c["Q"], c["x"], c["E_k"], c["E_v"], c["W"], c["rhos"], c["V"],
                               c["unique"], Cb, O, LSE, c["dO"])
    if timers is not None:
        timers["bwd"][1].record()
    return grads


def cpu_baseline_attention(c, seconds=15.0):
    """The oracle's fp32 restatement of the reference attention (sparse form with the
    absent-slot mass, which equals the dense flash_ema_attention.py path), forward and
    reference backward formulas, on a slice of sequence 0 of the same batch: as many
    leading steps as fit in about `seconds` (at least 16)."""
    from oracle import attention as att
    from oracle import scan as oscan
    d = c["cpu"]
    H, hd, N, V = c["H"], c["hd"], c["N"], c["V"]
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(123)
    K = int(d["counts"][0])
    uniq = d["unique"][:1, :K]
    cb = d["c_base"][:1, :K]
    Ek = torch.randn(1, K, H * hd, generator=g) * 0.02
    Ev = torch.randn(1, K, H * hd, generator=g) * 0.02
    W = torch.randn(N, H * hd, generator=g) * 0.02
    steps, done_steps, elapsed = 16, 0, 0.0
    while True:
        x = d["x"][:1, :steps]
        Q = torch.randn(1, H, steps, hd, generator=g) * 0.02
        dO = torch.randn(1, H, steps, hd, generator=g)
        t = time.perf_counter()
        att.sparse_backward_formulas(Q, x, Ek, Ev, W, d["rhos"], V, uniq, dO, cb)
        elapsed = time.perf_counter() - t
        done_steps = steps
        if elapsed > seconds / 4 or steps >= c["L"]:
            break
        steps = min(c["L"], steps * 2)
    return {"value": done_steps / elapsed, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": (f"sequence 0 of the batch (K_b={K} slots), first {done_steps} steps, "
                       f"forward + reference backward formulas in torch fp32 on {cores} threads; "
                       f"{elapsed:.1f} s")}


def run_attention(args):
    c = attention_case()
    for _ in range(args.warmup):
        attention_step(c)
    torch.cuda.synchronize()
    timers_all = []
    t0, t1 = _events()
    torch.cuda.synchronize()
    t0.record()
    for _ in range(args.steps):
        timers = {"fwd": _events(), "bwd": _events()}
        attention_step(c, timers)
        timers_all.append(timers)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    fwd_ms = sum(t["fwd"][0].elapsed_time(t["fwd"][1]) for t in timers_all) / args.steps
    bwd_ms = sum(t["bwd"][0].elapsed_time(t["bwd"][1]) for t in timers_all) / args.steps
    L, N, D = c["L"], c["N"], c["D"]
    pairs = int(c["counts"].sum()) * L          # valid (t, k) pairs
    fwd_flop = pairs * (2 * N * D + 4 * D)
    bwd_flop = pairs * (4 * N * D + 10 * D)
    tokens = c["B"] * L
    bwd_tflops = bwd_flop / (bwd_ms * 1e-3) / 1e12
    line = {
        "metric": "flash-EMA attn fwd+bwd tokens/s at B56 T512 d512 N64; % MFMA/HBM peak",
        "value": round(tokens / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 gate MFMA, fp32 state/softmax/accumulate",
        "data": "synthetic Zipf(1.1) tokens, seeded; random N(0,0.02) weights",
        "config": {"workload": "cfg2: one flash-EMA layer fwd+bwd (boundary states + fwd + bwd)",
                   "B": c["B"], "T": L, "d_model": D, "heads": c["H"], "head_dim": c["hd"],
                   "N": N, "V": c["V"], "K_max": c["K"], "sum_K_b": int(c["counts"].sum()),
                   "fwd_ms": round(fwd_ms, 4), "bwd_ms": round(bwd_ms, 4),
                   "fwd_bwd_tflops": round((fwd_flop + bwd_flop) / ((fwd_ms + bwd_ms) * 1e-3) / 1e12, 2),
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "kernel": "flash_ema_bwd_kernel",
                     "achieved": round(bwd_tflops, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(bwd_tflops / PEAK_BF16_TFLOPS, 4),
                     "traffic": TRAFFIC_BYTES.get("flash_ema_bwd_kernel")},
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_attention(c)
    return line


def run_scan(args):
    from mathbrain_amd.ema_query import compute_query_ema_history
    from mathbrain_amd.synthetic import make_batch
    B, T, N, V = 56, 2048, 128, 50257
    d = make_batch(B, T, V, N, 8192, seed=3)
    dev = torch.device("cuda", torch.cuda.current_device())
    x, rh, cb, u = (d[k].to(dev) for k in ("x", "rhos", "c_base", "unique"))
    # rotate 4 input copies so consecutive calls do not hit the previous call's lines
    xs = [x.clone() for _ in range(4)]
    for i in range(args.warmup):
        compute_query_ema_history(xs[i % 4], rh, V, cb, u, return_state=True)
    torch.cuda.synchronize()
    t0, t1 = _events()
    t0.record()
    for i in range(args.steps):
        compute_query_ema_history(xs[i % 4], rh, V, cb, u, return_state=True)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    # x + C_seq + touched c_base rows read + lazy state written + stamps
    touched = 0
    for b in range(B):
        touched += int(torch.isin(d["unique"][b, :d["counts"][b]], d["x"][b]).sum())
    nbytes = B * T * 8 + B * T * N * 4 + 2 * touched * N * 4 + touched * 4
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {
        "metric": "EMA query scan GB/s (cfg3: B56 T2048 N128 V50257)",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
        "config": {"workload": "cfg3 EMA query scan with final lazy state", "B": B, "T": T,
                   "N": N, "V": V, "bytes_per_call": nbytes},
        "roofline": {"bound": "hbm", "kernel": "ema_query_scan_kernel", "achieved": round(gbs, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                     "traffic": None},
    }


def run_copy(args):
    n = (1 << 30) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(args.warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    t0, t1 = _events()
    t0.record()
    for _ in range(args.steps):
        dst.copy_(src)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    gbs = 2 * n * 4 / (ms * 1e-3) / 1e9
    return {"metric": "device copy GB/s (1 GiB read + 1 GiB written)", "value": round(gbs, 1),
            "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
            "config": {"workload": "reference copy for counter scaling", "bytes_read": n * 4,
                       "bytes_written": n * 4}}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=("attention", "scan", "copy"), default="attention")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(sharding across GPUs is described in DESIGN.md, not run)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs an MI355X GPU", file=sys.stderr)
        sys.exit(1)
    run = {"attention": run_attention, "scan": run_scan, "copy": run_copy}[args.workload]
    line = run(args)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
