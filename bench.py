"""Benchmark of the Per-Slot EMA hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload attention|cfg4|scan|gating|model|copy|corpus|batch|factored]

Default workload (configuration 2 of the task): one flash-EMA gated attention layer,
forward + backward, B=56, T=512, d_model=512, 8 heads x 64, N=64 EMA rates, V=50257,
Zipf(1.1) tokens, c_base from a 4096-token warm-up per sequence, weights N(0, 0.02),
dO N(0, 1) (synthetic, seeded).  One step = key-side chunk states (mb_ema_boundary_states)
+ forward (mb_flash_ema_fwd) + backward (mb_flash_ema_bwd), all inputs resident in HBM.

Prints one JSON line.  `roofline` is for the dominant kernel (the backward): algorithmic
flops per launch, sum_b L*K_b*(4*N*D + 10*D) (gate recompute, dW_pe and five
per-element products: dO . (e_v g), dQ, dE_k, dE_v and dpre; the scores come from the
forward, as FlashEMAFunction keeps them; only valid (t, k) pairs count), over its mean launch
time measured with HIP events on the launch stream, against the dense bf16/fp16 MFMA peak of 2516.6 TFLOP/s.
`cpu_baseline` times the CPU restatement of the reference algorithm (the oracle, a port
of the reference's PyTorch path) on a bounded slice of the same workload on this host.

After the headline measurement the default run adds `secondary`: the cfg3 query scan, the
query gating at cfg2's rows, the cfg4 attention step and the cfg5 training step, each measured the way its own
`--workload` measures it (fewer steps, no CPU baseline); `--no-secondary` skips them.

`--workload cfg4` runs the same step at configuration 4 (B=16, T=4096, N=128, a random
0-10 % tail of padding per sequence with dO zero there); it is a second measurement, not the
headline metric.
`--workload scan` measures the EMA query scan of configuration 3 instead (B=56, T=2048,
N=128, c_base from an 8192-token warm-up) in GB/s of algorithmic traffic.
`--workload gating` measures the query gating forward + backward (mb_gating_fwd/bwd with
pe_proj folded in) at configuration 2's rows (B=56, T=512, D=512, N=64) in GB/s.
`--workload model` runs configuration 5: a full SlotTransformerLM training step (6 layers,
d_model 512, 8 heads, N=64, V=50257, B=56, T=512, bf16 autocast, AdamW, gradient
clipping) on chunks of synthetic lognormal-length Zipf documents with carried c_base.
`--workload copy` runs a plain 1 GiB device-to-device copy: the reference dispatch that
scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters to bytes.
`--workload corpus` runs the corpus EMA state scan of preprocess_corpus (mb_corpus_states)
over a 64 M-token synthetic corpus, and `--workload batch` the device batch builder
(mb_slot_lists + mb_slot_batch) on 56 chunks of 513 tokens with history-expanded slots and
c_base; both in tokens/s with an HBM roofline.
`--workload factored` runs the factored linear EMA (factored_ema_forward + backward) at
configuration 2's shapes with c_base, against the fp32 peak.
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

# HBM bytes per backward (its flash_ema_bwd_kernel dispatches), from the rocprofv3
# FETCH_SIZE and WRITE_SIZE passes scaled by a 1 GiB copy (profiles/flash_ema_cfg2.md,
# profiles/flash_ema_cfg4.md); re-measured whenever the kernel changes.
# the attention's arithmetic per --precision (the default splits the gate operands where
# N <= 64 and head_dim <= 64, and takes single fp16 operands beyond)
GATE_DTYPES = {
    "bf16": ("fp16 hi+lo split gate MFMA (3 products on the large-counter rate tile, 1 on the other; "
             "in the backward only for slots whose stored p reaches 2^-7, else 1 product), bf16 dW_pe "
             "MFMA, fp32 state/softmax/accumulate"),
    "fp16": "fp16 gate MFMA (1 product), bf16 dW_pe MFMA, fp32 state/softmax/accumulate",
    "fp32": "fp32 mode: fp16 hi+lo gate MFMA (bf16 hi+lo dW_pe MFMA), fp32 state/softmax/accumulate",
}

TRAFFIC_BYTES = {
    "cfg2": 14703.6e6,     # flash_ema_bwd_kernel, default mode (profiles/flash_ema_cfg2.md)
    "cfg4": 50700.7e6,
    "corpus": 19654.0e6,   # the three mb_corpus_states launches (profiles/corpus_states_64M_tokens.md)
    "scan": 109.3e6,       # ema_query_scan_kernel at configuration 3 (profiles/ema_query_scan_cfg3.md)
    "gating": 484.0e6,     # gating_fwd_rows_kernel + gating_bwd_rows_kernel (profiles/gating_cfg2_rows.md)
}


def _events():
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def _cpu_model():
    """The host CPU's model name (what lscpu prints), from /proc/cpuinfo."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


ATTENTION_CONFIGS = {
    # name: (B, T, heads, head_dim, N, V, padding tail fraction)
    "cfg2": (56, 512, 8, 64, 64, 50257, 0.0),
    "cfg4": (16, 4096, 8, 64, 128, 50257, 0.1),
}


def attention_case(seed=0, config="cfg2"):
    from mathbrain.synthetic import make_batch
    B, L, H, hd, N, V, pad = ATTENTION_CONFIGS[config]
    d = make_batch(B, L, V, N, 4096, seed=seed, pad_frac=pad)
    dev = torch.device("cuda", torch.cuda.current_device())
    g = torch.Generator().manual_seed(seed + 1)
    K = d["unique"].shape[1]
    D = H * hd
    c = dict(B=B, L=L, H=H, hd=hd, N=N, V=V, K=K, D=D, counts=d["counts"], config=config)
    c["x"] = d["x"].to(dev)
    c["unique"] = d["unique"].to(dev)
    c["c_base"] = d["c_base"].to(dev)
    c["rhos"] = d["rhos"].to(dev)
    c["Q"] = (torch.randn(B, H, L, hd, generator=g) * 0.02).to(dev)
    c["E_k"] = (torch.randn(B, K, D, generator=g) * 0.02).to(dev)
    c["E_v"] = (torch.randn(B, K, D, generator=g) * 0.02).to(dev)
    c["W"] = (torch.randn(N, D, generator=g) * 0.02).to(dev)
    dO = torch.randn(B, H, L, hd, generator=g)
    for b in range(B):                 # the loss is masked on the padding tail
        if d["pad_len"][b] > 0:
            dO[b, :, L - int(d["pad_len"][b]):] = 0
    c["dO"] = dO.to(dev)
    c["cpu"] = d
    return c


def attention_step(c, timers=None, precision="bf16"):
    from mathbrain.triton_flash_ema import (_forward_with_scores, _prec, flash_ema_backward,
                                            flash_ema_forward, keep_scores, precompute_boundaries)
    # the forward keeps its scores for the backward when FlashEMAFunction would (the same
    # call FlashEMAFunction makes then)
    keep = keep_scores(c["B"], c["H"], c["K"], c["L"])
    Cb = precompute_boundaries(c["x"], c["unique"], c["rhos"], 64, c["c_base"])
    if timers is not None:
        timers["fwd"][0].record()
    if keep:
        res = _forward_with_scores(c["Q"], c["x"], c["E_k"], c["E_v"], c["W"], c["rhos"], c["V"],
                                   c["unique"], Cb, True, 64, True, _prec(precision))
    else:
        res = flash_ema_forward(c["Q"], c["x"], c["E_k"], c["E_v"], c["W"], c["rhos"], c["V"],
                                c["unique"], c["K"], Cb, precision=precision)
    O, LSE = res[0], res[1]
    if timers is not None:
        timers["fwd"][1].record()
        timers["bwd"][0].record()
    grads = flash_ema_backward(c["Q"], c["x"], c["E_k"], c["E_v"], c["W"], c["rhos"], c["V"],
                               c["unique"], Cb, O, LSE, c["dO"], precision=precision,
                               scores=res[5] if keep else None)
    if timers is not None:
        timers["bwd"][1].record()
    return grads


def cpu_baseline_attention(c, seconds=12.0):
    """The oracle's fp32 restatement of the reference attention (sparse form with the
    absent-slot mass, which equals the dense flash_ema_attention.py path), forward and
    reference backward formulas, on whole sequences of the same batch (all L steps,
    each with its own K_b slots), one after another until about `seconds` have passed."""
    from oracle import attention as att
    d = c["cpu"]
    H, hd, N, V, L = c["H"], c["hd"], c["N"], c["V"], c["L"]
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(123)
    W = torch.randn(N, H * hd, generator=g) * 0.02
    done, elapsed, slots = 0, 0.0, []
    for b in range(c["B"]):
        K = int(d["counts"][b])
        uniq = d["unique"][b:b + 1, :K]
        cb = d["c_base"][b:b + 1, :K]
        Ek = torch.randn(1, K, H * hd, generator=g) * 0.02
        Ev = torch.randn(1, K, H * hd, generator=g) * 0.02
        Q = torch.randn(1, H, L, hd, generator=g) * 0.02
        dO = torch.randn(1, H, L, hd, generator=g)
        t = time.perf_counter()
        att.sparse_backward_formulas(Q, d["x"][b:b + 1], Ek, Ev, W, d["rhos"], V, uniq, dO, cb)
        elapsed += time.perf_counter() - t
        done += L
        slots.append(K)
        if elapsed > seconds:
            break
    return {"value": done / elapsed, "unit": "tokens/s", "cores": cores, "kind": "port",
            "cpu_model": _cpu_model(),
            "sample": (f"sequences 0..{len(slots) - 1} of the batch (K_b = {min(slots)}..{max(slots)} "
                       f"slots), all {L} steps each, forward + reference backward formulas in "
                       f"torch fp32 on {cores} threads; {elapsed:.1f} s")}


def cpu_baseline_dense_forward(c, steps=12):
    """The reference's dense all-vocabulary CPU forward (flash_ema_attention.py:19-85, the
    oracle's restatement) on the first `steps` steps of one sequence.  Its work per step is
    the same at every step and for every sequence (decay, gate and attend over all V slots),
    so tokens/s is extrapolated from that sample to the whole batch; it has no backward (the
    reference's in-place update blocks autograd)."""
    from oracle import attention as att
    d = c["cpu"]
    H, hd, N, V = c["H"], c["hd"], c["N"], c["V"]
    D = H * hd
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(321)
    Q = torch.randn(1, steps, D, generator=g) * 0.02
    Ek = torch.randn(V, D, generator=g) * 0.02
    Ev = torch.randn(V, D, generator=g) * 0.02
    Wp = torch.randn(D, N, generator=g) * 0.02
    att.dense(Q[:, :1], d["x"][:1, :1], Ek, Ev, d["rhos"], Wp, H)   # warm-up step
    t = time.perf_counter()
    att.dense(Q, d["x"][:1, :steps], Ek, Ev, d["rhos"], Wp, H)
    sec = time.perf_counter() - t
    return {"value": round(steps / sec, 2), "unit": "tokens/s", "cores": cores, "kind": "port",
            "cpu_model": _cpu_model(), "extrapolated": True,
            "sample": (f"dense all-vocabulary forward only (V={V}, fp32, {cores} threads), the first "
                       f"{steps} steps of sequence 0 in {sec:.1f} s; per-step work is constant, so the "
                       f"rate is extrapolated to the B={c['B']}, T={c['L']} batch")}


def run_attention(args):
    c = attention_case(config="cfg4" if args.workload == "cfg4" else "cfg2")
    for _ in range(args.warmup):
        attention_step(c, precision=args.precision)
    torch.cuda.synchronize()
    timers_all = []
    t0, t1 = _events()
    torch.cuda.synchronize()
    t0.record()
    for _ in range(args.steps):
        timers = {"fwd": _events(), "bwd": _events()}
        attention_step(c, timers, args.precision)
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
    if c["config"] == "cfg2":
        metric = "flash-EMA attn fwd+bwd tokens/s at B56 T512 d512 N64; % MFMA/HBM peak"
        workload = "cfg2: one flash-EMA layer fwd+bwd (boundary states + fwd + bwd)"
    else:
        metric = "flash-EMA attn fwd+bwd tokens/s at B16 T4096 d512 N128 (configuration 4)"
        workload = ("cfg4: one flash-EMA layer fwd+bwd (boundary states + fwd + bwd), "
                    "0-10 % padding tail per sequence")
    line = {
        "metric": metric,
        "value": round(tokens / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": GATE_DTYPES[args.precision] if N <= 64 or args.precision != "bf16" else GATE_DTYPES["fp16"],
        "data": "synthetic Zipf(1.1) tokens, seeded; random N(0,0.02) weights",
        "config": {"workload": workload,
                   "B": c["B"], "T": L, "d_model": D, "heads": c["H"], "head_dim": c["hd"],
                   "N": N, "V": c["V"], "K_max": c["K"], "sum_K_b": int(c["counts"].sum()),
                   "fwd_ms": round(fwd_ms, 4), "bwd_ms": round(bwd_ms, 4),
                   "fwd_bwd_tflops": round((fwd_flop + bwd_flop) / ((fwd_ms + bwd_ms) * 1e-3) / 1e12, 2),
                   "precision": args.precision, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "kernel": "flash_ema_bwd_kernel",
                     "achieved": round(bwd_tflops, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(bwd_tflops / PEAK_BF16_TFLOPS, 4),
                     "traffic": TRAFFIC_BYTES.get(c["config"]) if args.precision == "bf16" else None},
    }
    if not args.no_cpu_baseline and c["config"] == "cfg2":
        # (at cfg4 one whole sequence alone takes the oracle minutes)
        line["cpu_baseline"] = cpu_baseline_attention(c)
        line["cpu_baseline_dense_forward"] = cpu_baseline_dense_forward(c)
    return line


def run_scan(args):
    from mathbrain import _lib
    from mathbrain.triton_ema_query import compute_query_ema_history
    from mathbrain.synthetic import make_batch
    B, T, N, V = 56, 2048, 128, 50257
    d = make_batch(B, T, V, N, 8192, seed=3)
    dev = torch.device("cuda", torch.cuda.current_device())
    K = d["unique"].shape[1]
    rh = d["rhos"].to(dev)
    u = d["unique"].to(dev)
    # four input/output sets, rotated, so consecutive calls miss the 256 MB MALL
    sets = []
    for _ in range(4):
        cb = d["c_base"].to(dev)
        sets.append(dict(x=d["x"].to(dev), cb=cb, out=torch.empty(B, T, N, device=dev),
                         state=cb.clone(), stamps=torch.empty(B, K, dtype=torch.int32, device=dev)))
    st = _lib.stream(dev)

    def call(s):
        _lib.call("mb_ema_query_scan", _lib.ptr(s["x"]), T, 1, B, T, _lib.ptr(rh), N, V,
                  _lib.ptr(s["cb"]), _lib.ptr(u), K, None, _lib.ptr(s["out"]), _lib.ptr(s["state"]),
                  _lib.ptr(s["stamps"]), st)

    for i in range(args.warmup):
        call(sets[i % 4])
    torch.cuda.synchronize()
    t0, t1 = _events()
    t0.record()
    for i in range(args.steps):
        call(sets[i % 4])
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    # the Python entry point on top (allocations, and a copy of c_init for the state)
    for i in range(2):
        compute_query_ema_history(sets[i]["x"], rh, V, sets[i]["cb"], u, return_state=True)
    torch.cuda.synchronize()
    w0, w1 = _events()
    w0.record()
    for i in range(args.steps):
        compute_query_ema_history(sets[i % 4]["x"], rh, V, sets[i % 4]["cb"], u, return_state=True)
    w1.record()
    torch.cuda.synchronize()
    wrapper_ms = w0.elapsed_time(w1) / args.steps
    # x + C_seq + touched c_base rows read + lazy state written + stamps
    touched = 0
    for b in range(B):
        touched += int(torch.isin(d["unique"][b, :d["counts"][b]], d["x"][b]).sum())
    nbytes = B * T * 8 + B * T * N * 4 + 2 * touched * N * 4 + touched * 4
    gbs = nbytes / (ms * 1e-3) / 1e9
    line = {
        "metric": "EMA query scan GB/s (cfg3: B56 T2048 N128 V50257)",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
        "config": {"workload": "cfg3 EMA query scan with final lazy state (C-ABI call, outputs "
                               "preallocated)", "B": B, "T": T, "N": N, "V": V,
                   "bytes_per_call": nbytes, "python_entry_ms": round(wrapper_ms, 4)},
        "roofline": {"bound": "hbm", "kernel": "ema_query_scan_kernel", "achieved": round(gbs, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                     "traffic": TRAFFIC_BYTES["scan"]},
    }
    if not args.no_cpu_baseline:
        # the reference's CPU scan (dense per-vocabulary tables, a loop over T vectorised over
        # B: triton_ema_query.py:67-117) on the whole configuration, as the oracle restates it
        from oracle import scan as oscan
        cores = len(os.sched_getaffinity(0))
        torch.set_num_threads(cores)
        c0 = time.perf_counter()
        oscan.query_scan_dense_loop(d["x"], d["rhos"], V, d["c_base"], d["unique"])
        sec = time.perf_counter() - c0
        line["cpu_baseline"] = {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "cores": cores,
                                "kind": "port", "cpu_model": _cpu_model(),
                                "sample": (f"the whole configuration (B={B}, T={T}, N={N}, V={V}) "
                                           f"through the reference's dense-table loop in torch fp32 "
                                           f"on {cores} threads: {sec:.2f} s, {B * T / sec:.0f} tokens/s; "
                                           f"value = the same algorithmic bytes over that time")}
    return line


def run_gating(args):
    from mathbrain import _lib
    B, L, D, N = 56, 512, 512, 64
    dev = torch.device("cuda", torch.cuda.current_device())
    g = torch.Generator().manual_seed(0)
    rows = B * L
    x_q = torch.randn(rows, D, generator=g).to(dev)
    C = (torch.rand(rows, N, generator=g) * 50).to(dev)
    W = (torch.randn(N, D, generator=g) * 0.02).to(dev)
    ln_w = torch.ones(D, device=dev)
    ln_b = torch.zeros(D, device=dev)
    dy = torch.randn(rows, D, generator=g).to(dev)
    y, dxq, dpre = (torch.empty(rows, D, device=dev) for _ in range(3))
    mu, rstd = torch.empty(rows, device=dev), torch.empty(rows, device=dev)
    col = [torch.empty(D, device=dev) for _ in range(3)]
    st = _lib.stream(dev)

    pre = torch.empty(rows, D, device=dev)

    # as GatedQueryFunction runs them: the forward keeps the pre-activation, the backward
    # takes it as p_pre (no bias) instead of recomputing the projection
    def fwd():
        _lib.call("mb_gating_fwd", _lib.ptr(x_q), D, None, 0, None, _lib.ptr(C), N, _lib.ptr(W), N,
                  _lib.ptr(ln_w), _lib.ptr(ln_b), rows, D, 1, 1e-5, _lib.ptr(y), _lib.ptr(mu),
                  _lib.ptr(rstd), _lib.ptr(pre), st)

    def bwd():
        _lib.call("mb_gating_bwd", _lib.ptr(dy), _lib.ptr(x_q), D, _lib.ptr(pre), D, None, None, 0,
                  None, 0, _lib.ptr(ln_w), _lib.ptr(mu), _lib.ptr(rstd), rows, D, 1,
                  _lib.ptr(dxq), _lib.ptr(dpre), *(_lib.ptr(t) for t in col), st)

    for _ in range(args.warmup):
        fwd()
        bwd()
    torch.cuda.synchronize()
    ev = [_events() for _ in range(2)]
    f_ms = b_ms = 0.0
    for _ in range(args.steps):
        ev[0][0].record(); fwd(); ev[0][1].record()
        ev[1][0].record(); bwd(); ev[1][1].record()
        torch.cuda.synchronize()
        f_ms += ev[0][0].elapsed_time(ev[0][1])
        b_ms += ev[1][0].elapsed_time(ev[1][1])
    f_ms /= args.steps
    b_ms /= args.steps
    # algorithmic bytes: fwd reads x_q, C, writes y, mu, rstd and the kept pre-activation;
    # bwd reads dy, x_q, pre, mu, rstd, writes dx_q and dpre
    fb = rows * (D * 4 * 3 + N * 4 + 8)
    bb = rows * (D * 4 * 5 + 8)
    gbs = (fb + bb) / ((f_ms + b_ms) * 1e-3) / 1e9
    return {"metric": "query gating fwd+bwd GB/s (cfg2 rows: B56 T512 D512 N64)", "value": round(gbs, 1),
            "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(f_ms + b_ms, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
            "config": {"workload": "gating fwd+bwd, pe_proj folded in, pre-activation kept for the backward", "rows": rows, "D": D, "N": N,
                       "fwd_ms": round(f_ms, 4), "bwd_ms": round(b_ms, 4)},
            "roofline": {"bound": "hbm", "kernel": "gating_fwd_rows_kernel + gating_bwd_rows_kernel",
                         "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": TRAFFIC_BYTES["gating"]}}


def run_model(args):
    import torch.nn.functional as F
    from mathbrain.model import SlotTransformerLM
    from mathbrain.synthetic import make_doc_batch
    B, T, V, N, D, n_layers, H = 56, 512, 50257, 64, 512, 6, 8
    dev = torch.device("cuda", torch.cuda.current_device())
    torch.set_float32_matmul_precision("high")   # train.py:94-95
    d = make_doc_batch(B, T, V, N, min_hl=1.0, max_hl=2048.0, seed=0)
    torch.manual_seed(1)
    model = SlotTransformerLM(V, D, n_layers, H, N=N, dropout=0.1, attn_precision=args.precision).to(dev)
    if args.fold_query_gating:  # queries inside the attention kernel (off by default)
        for layer in model.layers:
            layer.attn.fold_query_gating = True
    # train.py:245-253: AdamW with weight decay 0.01 and a linear warmup over the first 200
    # steps (the cosine decay after it is never reached by a benchmark run)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-3, weight_decay=0.01)
    sched = torch.optim.lr_scheduler.LambdaLR(opt, lambda s: s / 200 if s < 200 else 1.0)
    x, uniq, cb, tgt = (d[k].to(dev) for k in ("x", "unique", "c_base", "targets"))
    pm = uniq >= 0

    def step():
        opt.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            logits = model(x, unique_slots=uniq, c_base=cb, pad_mask=pm)
            loss = F.cross_entropy(logits.view(-1, V), tgt.view(-1), ignore_index=-1)
        loss.backward()
        torch.nn.utils.clip_grad_norm_(model.parameters(), 1.0)
        opt.step()
        sched.step()
        return loss

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0, t1 = _events()
    t0.record()
    for _ in range(args.steps):
        loss = step()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    n_params = sum(p.numel() for p in model.parameters())
    real = int((tgt >= 0).sum())
    return {"metric": "SlotTransformerLM training step tokens/s (cfg5)", "value": round(B * T / (ms * 1e-3), 1),
            "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(ms, 3), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None,
            "dtype": "bf16 autocast; attention: " + GATE_DTYPES[args.precision],
            "data": "synthetic lognormal(median 1500) Zipf(1.1) documents, chunked, random init",
            "config": {"workload": "cfg5 full training step", "layers": n_layers, "d_model": D,
                       "heads": H, "N": N, "V": V, "B": B, "T": T, "params": n_params,
                       "K_max": int(uniq.shape[1]), "unpadded_tokens": real,
                       "steps_per_s": round(1e3 / ms, 3),
                       "unpadded_tokens_per_s": round(real / (ms * 1e-3), 1),
                       "query_gating": "inside the attention kernel" if args.fold_query_gating
                                       else "separate kernel + q_proj GEMM",
                       "loss": round(float(loss), 4)}}


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


def run_corpus(args):
    """The corpus state scan of preprocess_corpus (mb_corpus_states) over a 64 M-token
    synthetic corpus (50257 ids, Zipf(1.1), lognormal documents of median 3000, N=64)."""
    import numpy as np
    from mathbrain import _lib
    from mathbrain.data import chain_order, corpus_states
    from mathbrain.synthetic import zipf_corpus
    T, V, N = 1 << 26, 50257, 64
    tokens, doc_ids = zipf_corpus(T, V, median_len=3000, seed=11)
    dev = torch.device("cuda", torch.cuda.current_device())
    rh = torch.exp(-math.log(2.0) / torch.logspace(0.0, math.log10(2048.0), N, dtype=torch.float64)
                   ).to(torch.float32).to(dev)
    tok, docs = torch.from_numpy(tokens).to(dev), torch.from_numpy(doc_ids).to(dev)
    chain, order = chain_order(tok, docs)
    states = torch.empty(T, N, dtype=torch.float32, device=dev)
    ws = int(_lib.lib().mb_corpus_states_workspace(T, N))
    work = torch.empty(ws, dtype=torch.uint8, device=dev)
    st = _lib.stream(dev)

    def call():
        _lib.call("mb_corpus_states", _lib.ptr(order), _lib.ptr(chain), T, _lib.ptr(rh), N,
                  _lib.ptr(states), _lib.ptr(work), ws, st)

    for _ in range(args.warmup):
        call()
    torch.cuda.synchronize()
    t0, t1 = _events()
    t0.record()
    for _ in range(args.steps):
        call()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    w0, w1 = _events()
    w0.record()
    corpus_states(tok, docs, rh)          # with the (segment, token) sort and allocations
    w1.record()
    torch.cuda.synchronize()
    wrapper_ms = w0.elapsed_time(w1)
    # algorithmic bytes: the sorted positions and keys read once, one state row written per
    # position
    nbytes = T * (16 + 4 * N)
    gbs = nbytes / (ms * 1e-3) / 1e9
    line = {
        "metric": "corpus EMA state scan tokens/s (preprocess_corpus, T=64M, N=64)",
        "value": round(T / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
        "config": {"workload": "corpus state scan (C-ABI call on the sorted chains, outputs "
                               "preallocated)", "T": T, "V": V, "N": N,
                   "bytes_per_call": nbytes, "python_entry_ms_with_sort": round(wrapper_ms, 3)},
        "roofline": {"bound": "hbm", "kernel": "mb_corpus_states (its 3 launches)",
                     "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": TRAFFIC_BYTES["corpus"]},
    }
    if not args.no_cpu_baseline:
        from oracle import data as od
        n = 1 << 22
        c0 = time.perf_counter()
        od.corpus_states(tokens[:n], doc_ids[:n], rh.cpu().numpy())
        sec = time.perf_counter() - c0
        line["cpu_baseline"] = {"value": round(n / sec, 1), "unit": "tokens/s", "cores": 1,
                                "kind": "port", "cpu_model": _cpu_model(),
                                "sample": "the first 2^22 tokens of the same corpus, data.py:276-303 "
                                          f"per-token loop in numpy ({sec:.1f} s)"}
    return line


def run_batch(args):
    """The batch builder (mb_slot_lists + mb_slot_batch): 56 chunks of 512 + 1 tokens of a
    16 M-token synthetic corpus (50257 ids, lognormal documents of median 4000, N=64),
    slots expanded with each document's history and c_base gathered from the state rows."""
    import numpy as np
    from mathbrain import _lib
    from mathbrain.data import chunk_index, corpus_states, next_occurrence
    from mathbrain.synthetic import zipf_corpus
    T, V, N, B, block = 1 << 24, 50257, 64, 56, 512
    tokens, doc_ids = zipf_corpus(T, V, median_len=4000, seed=12)
    dev = torch.device("cuda", torch.cuda.current_device())
    rh = torch.exp(-math.log(2.0) / torch.logspace(0.0, math.log10(2048.0), N, dtype=torch.float64)
                   ).to(torch.float32).to(dev)
    tok, docs = torch.from_numpy(tokens).to(dev), torch.from_numpy(doc_ids).to(dev)
    states = corpus_states(tok, docs, rh)
    nxt = next_occurrence(tok)
    cs, ce, cd, starts = chunk_index(doc_ids, block)
    cds = np.asarray([starts[int(d)] for d in cd], np.int64)
    rng = np.random.default_rng(0)
    sets = []
    for _ in range(8):
        idx = rng.choice(len(cs), size=B, replace=False)
        desc = torch.from_numpy(np.stack([cds[idx], cs[idx], ce[idx]])).to(dev)
        sets.append((idx, desc, int((ce[idx] - cs[idx]).max())))
    tabs = dict(last=torch.empty(B, V, dtype=torch.int32, device=dev),
                slot_of=torch.empty(B, V, dtype=torch.int32, device=dev),
                slot_tok=torch.empty(B, V, dtype=torch.int64, device=dev),
                counts=torch.empty(B, 2, dtype=torch.int32, device=dev))
    st = _lib.stream(dev)
    P = _lib.ptr

    def lists(desc):
        _lib.call("mb_slot_lists", P(tok), P(nxt), T, V, P(desc[0]), P(desc[1]), P(desc[2]), B,
                  P(tabs["last"]), P(tabs["slot_of"]), P(tabs["slot_tok"]), P(tabs["counts"]), st)

    kmax = []
    for _, desc, _ in sets:
        lists(desc)
        kmax.append(int(tabs["counts"][:, 1].max()))
    K_max, L = max(kmax), max(x[2] for x in sets)
    out = dict(chunks=torch.empty(B, L, dtype=torch.int64, device=dev),
               docs=torch.empty(B, L, dtype=torch.int64, device=dev),
               inv=torch.empty(B, L, dtype=torch.int64, device=dev),
               slots=torch.empty(B, K_max, dtype=torch.int64, device=dev),
               mask=torch.empty(B, K_max, dtype=torch.bool, device=dev),
               c_base=torch.empty(B, K_max, N, dtype=torch.float32, device=dev))

    def call(i):
        desc = sets[i % len(sets)][1]
        lists(desc)
        _lib.call("mb_slot_batch", P(tok), P(docs), P(states), P(rh), N, T, V, P(desc[0]),
                  P(desc[1]), P(desc[2]), B, P(tabs["last"]), P(tabs["slot_of"]),
                  P(tabs["slot_tok"]), P(tabs["counts"]), L, K_max, P(out["chunks"]),
                  P(out["docs"]), P(out["slots"]), P(out["mask"]), P(out["inv"]),
                  P(out["c_base"]), st)

    for i in range(args.warmup):
        call(i)
    torch.cuda.synchronize()
    t0, t1 = _events()
    t0.record()
    for i in range(args.steps):
        call(i)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    # algorithmic bytes of one batch: the history and chunk tokens scanned (token + next
    # position), the state rows read and c_base written, the chunk rows and slot lists written
    span = sum(int((ce[x[0]] - cds[x[0]]).sum()) for x in sets) / len(sets)
    slots = sum(kmax) / len(kmax) * B
    nbytes = span * 8 + 2 * slots * N * 4 + B * L * 24 + B * K_max * 9
    gbs = nbytes / (ms * 1e-3) / 1e9
    line = {
        "metric": "slot batch builder tokens/s (56 chunks x 513 tokens, V=50257, N=64)",
        "value": round(B * L / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32 / int64",
        "data": "synthetic",
        "config": {"workload": "collated batch with history-expanded slots and c_base "
                               "(mb_slot_lists + mb_slot_batch, outputs preallocated)",
                   "B": B, "L": L, "V": V, "N": N, "corpus_tokens": T, "mean_slots": round(slots / B, 1),
                   "K_max": K_max, "mean_doc_prefix_scanned": round(span / B, 1),
                   "bytes_per_call": int(nbytes)},
        "roofline": {"bound": "hbm", "kernel": "mb_slot_lists + mb_slot_batch (their 5 launches)",
                     "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None},
    }
    if not args.no_cpu_baseline:
        from oracle import data as od
        rhn = rh.cpu().numpy()
        st_h = states.cpu().numpy()
        pos = {}
        order = np.argsort(tokens, kind="stable").astype(np.int32)
        srt = tokens[order]
        cuts = np.flatnonzero(srt[1:] != srt[:-1]) + 1
        pos = {int(k): p for k, p in zip(srt[np.concatenate([[0], cuts])], np.split(order, cuts))}
        c0 = time.perf_counter()
        ntok, nb = 0, 0
        while nb < len(sets) and time.perf_counter() - c0 < 10.0:
            idx = sets[nb][0]
            items = [od.get_item(tokens, doc_ids, st_h, pos, starts,
                                 (int(cs[i]), int(ce[i]), int(cd[i])), rhn) for i in idx]
            od.collate(items)
            ntok += B * int((ce[idx] - cs[idx]).max())
            nb += 1
        sec = time.perf_counter() - c0
        line["cpu_baseline"] = {"value": round(ntok / sec, 1), "unit": "tokens/s", "cores": 1,
                                "kind": "port", "cpu_model": _cpu_model(),
                                "sample": f"{nb} of the timed batches, data.py:93-148 per-sample loop "
                                          f"+ collate in numpy ({sec:.1f} s)"}
    return line


def run_factored(args):
    """The factored linear EMA (factored_ema_forward, fwd + bwd) at configuration 2's shapes:
    B=56, T=512, d_model 512, 8 heads x 64, N=64, V=50257, c_base over the history-expanded
    slots of a 4096-token warm-up per sequence."""
    from mathbrain.factored_ema import factored_ema_forward
    from mathbrain.synthetic import make_batch
    B, T, H, hd, N, V = 56, 512, 8, 64, 64, 50257
    D = H * hd
    d = make_batch(B, T, V, N, 4096, min_hl=1.0, max_hl=4096.0, seed=0)
    dev = torch.device("cuda", torch.cuda.current_device())
    g = torch.Generator().manual_seed(1)
    Q = (torch.randn(B, T, D, generator=g) * 0.02).to(dev).requires_grad_(True)
    Ek = (torch.randn(V, D, generator=g) * 0.02).to(dev).requires_grad_(True)
    Ev = (torch.randn(V, D, generator=g) * 0.02).to(dev).requires_grad_(True)
    W = (torch.randn(N, D, generator=g) * 0.02).to(dev).requires_grad_(True)
    dO = torch.randn(B, T, D, generator=torch.Generator().manual_seed(2)).to(dev)
    x, u, cb, rh = d["x"].to(dev), d["unique"].to(dev), d["c_base"].to(dev), d["rhos"].to(dev)
    pm = u >= 0

    def step():
        for t in (Q, Ek, Ev, W):
            t.grad = None
        O = factored_ema_forward(Q, x, Ek, Ev, rh, W, H, c_base=cb, unique_slots=u, pad_mask=pm)
        O.backward(dO)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0, t1 = _events()
    t0.record()
    for _ in range(args.steps):
        step()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    K = int(d["counts"].sum())
    pairs = B * T * (T - 1) // 2
    # algorithmic flops: token pairs 23*hd (forward 5, backward 18), the c_base state built,
    # applied to the steps and to the slots (6 K N hd^2 + 6 T N hd^2 per sequence and head)
    flops = H * (pairs * 23 * hd + 6 * K * N * hd * hd + 6 * B * T * N * hd * hd)
    tf = flops / (ms * 1e-3) / 1e12
    line = {
        "metric": "factored linear EMA fwd+bwd tokens/s (cfg2 shapes: B56 T512 d512 H8x64 N64)",
        "value": round(B * T / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic Zipf(1.1) tokens, c_base from a 4096-token warm-up, weights N(0, 0.02)",
        "config": {"workload": "factored_ema_forward + backward (autograd, c_base state)",
                   "B": B, "T": T, "D": D, "H": H, "N": N, "V": V, "slots": K,
                   "algorithmic_tflop": round(flops / 1e12, 3)},
        "roofline": {"bound": "mfma", "kernel": "all factored kernels (token pairs fp32 VALU; "
                                               "state GEMMs bf16 MFMA on hi/lo-split fp32 operands)",
                     "achieved": round(tf, 2), "peak": 157.3, "unit": "TFLOP/s",
                     "frac": round(tf / 157.3, 4), "traffic": None},
    }
    if not args.no_cpu_baseline:
        from oracle import factored as of
        torch.set_num_threads(min(16, len(os.sched_getaffinity(0))))
        Tc = 128
        Qc = Q.detach().cpu()[:1, :Tc].clone().requires_grad_(True)
        Ekc = Ek.detach().cpu().requires_grad_(True)
        Evc = Ev.detach().cpu().requires_grad_(True)
        Wc = W.detach().cpu().requires_grad_(True)
        c0 = time.perf_counter()
        o = of.loop_forward(Qc, d["x"][:1, :Tc], Ekc, Evc, d["rhos"], Wc, H, c_base=d["c_base"][:1],
                            unique_slots=d["unique"][:1], pad_mask=d["unique"][:1] >= 0)
        o.backward(dO.cpu()[:1, :Tc])
        sec = time.perf_counter() - c0
        line["cpu_baseline"] = {"value": round(Tc / sec, 1), "unit": "tokens/s",
                                "cores": torch.get_num_threads(), "kind": "port", "cpu_model": _cpu_model(),
                                "sample": f"one sequence, its first {Tc} steps, factored_ema.py:22-96 "
                                          f"loop in torch fp32 + autograd backward ({sec:.1f} s)"}
    return line


def secondary(args):
    """The other configurations' numbers, measured in the same run after the headline one
    (its timed region is over): the cfg3 query scan, the query gating at cfg2's rows, the
    cfg4 attention step and the cfg5 training step, each its own workload's measurement at
    fewer steps and without a CPU baseline.  Each entry keeps that workload's value, unit, ms and roofline."""
    out = {}
    for name, fn, steps, workload in (("cfg3_scan", run_scan, 50, "scan"),
                                      ("gating_cfg2_rows", run_gating, 20, "gating"),
                                      ("cfg4_attention", run_attention, 3, "cfg4"),
                                      ("cfg5_training_step", run_model, 10, "model")):
        sub = argparse.Namespace(**vars(args))
        sub.steps, sub.warmup, sub.no_cpu_baseline = steps, 1 if workload == "cfg4" else 3, True
        sub.workload = workload
        r = fn(sub)
        entry = {"metric": r["metric"], "value": r["value"], "unit": r["unit"], "steps": steps,
                 "ms_per_step": r["ms_per_step"]}
        if "roofline" in r:
            entry["roofline"] = {k: r["roofline"][k] for k in ("kernel", "achieved", "unit", "frac")}
        out[name] = entry
        del r
        torch.cuda.empty_cache()
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=("attention", "cfg4", "scan", "gating", "model", "copy",
                                           "corpus", "batch", "factored"),
                    default="attention")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--precision", choices=("bf16", "fp16", "fp32"), default="bf16",
                    help="attention gate arithmetic (triton_flash_ema.PRECISIONS): split fp16 hi + lo "
                         "gate operands (bf16, the default), single fp16 operands (fp16), or the split "
                         "gate and a split dW_pe product (fp32); attention, cfg4 and model workloads")
    ap.add_argument("--no-secondary", action="store_true",
                    help="default workload: skip the secondary measurements (cfg3 scan, gating, cfg4, "
                         "cfg5 training step) that follow the headline one in the same run")
    ap.add_argument("--fold-query-gating", action="store_true",
                    help="model workload: compute the queries inside the attention kernel "
                         "(SlotAttentionLayer.fold_query_gating; off by default)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(how the path would shard is documented, not run)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs an MI355X GPU", file=sys.stderr)
        sys.exit(1)
    run = {"attention": run_attention, "cfg4": run_attention, "scan": run_scan,
           "gating": run_gating, "model": run_model, "copy": run_copy, "corpus": run_corpus,
           "batch": run_batch, "factored": run_factored}[args.workload]
    line = run(args)
    if args.workload == "attention" and not args.no_secondary:
        line["secondary"] = secondary(args)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
