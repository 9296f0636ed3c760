#!/usr/bin/env python3
"""Benchmark of the algebraic hot path on one MI355X (the BASELINE.json metric).

One step = the 1B-shape workload of BASELINE.json config 4, inputs resident in HBM:
  * causal algebraic attention forward + backward, B=8 H=16 T=2048 D=128 bf16, QK
    RMS-normalised, learned per-head sink, n=16 c=8, range_guard=True
    (the model's call, src/algebraic/model.py:145-150);
  * fused algebraic head forward + backward, N=16384 tokens, d=2048, V=32000 bf16,
    n=8 c=2 (src/algebraic/model.py:219-224).
FLOP conventions are the reference's: attention fwd 4 B H T^2 D / 2, fwd+bwd 3.5x
(scripts/bench_attention.py:50, 65); head 3 matmuls 3*2*N*d*V (scripts/bench_head.py:35).

Prints ONE JSON line. ``value`` is the step's algorithmic TFLOP/s (attention + head);
the attention TFLOP/s, the head tokens/s and each part's fraction of the bf16 dense MFMA
peak are reported beside it, with a roofline entry for the kernel that takes the most time
(per-kernel durations from HIP events recorded on the launch stream) and a CPU baseline
(the NumPy oracle timed on a bounded sample of the same workload on the host cores).
The other BASELINE configs (C1 attention fwd fp32, C2 head, C3 attention fwd+bwd D64, C5
long-context attention fwd) are timed as well (20 wrapper calls back to back, and the median of 20 single calls) and reported under
``other_configs``; they are not part of ``value``.
"""

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "algebraic-transformer_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "algebraic attn fwd+bwd TFLOP/s & head tokens/s at 1B shape; % MFMA peak"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA (no sparsity)
PEAK_HBM_GBS = 8000.0

ATTN = dict(B=8, H=16, T=2048, D=128, n=16, c=8.0)
HEAD = dict(N=16384, d=2048, V=32000, n=8, c=2.0)


def attn_flops(B, H, T, D, **_):
    return 4.0 * B * H * T * T * D / 2


def head_flops(N, d, V, **_):
    return 3.0 * 2.0 * N * d * V


def kernel_algorithmic_flops():
    """Algorithmic FLOPs per launch of each heavy kernel (units x per-unit figure)."""
    fa = attn_flops(**ATTN)
    g = 2.0 * HEAD["N"] * HEAD["d"] * HEAD["V"]   # one N x d x V product
    return {
        "attn_fwd_inrange": fa,          # QK^T + PV over the causal half
        "attn_bwd_inrange": 2.0 * fa,    # dK/dV kernel: S, dP, dV, dK
        "attn_bwd_dq_inrange": 1.5 * fa,  # dQ kernel: S and dP again, dQ
        "head_fwd": g,                   # z = h E^T
        "head_dz": g,                    # z recomputed (executed; the 3-matmul convention omits it)
        "head_dh": g,                    # dh = dZ E
        "head_de": g,                    # dE = dZ^T h
    }


def rms_norm(x, eps=1e-5):
    return x * (x.float().pow(2).mean(-1, keepdim=True) + eps).rsqrt().to(x.dtype)


def make_inputs(torch, dev, seed=0):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    B, H, T, D = (ATTN[k] for k in "BHTD")
    rn = lambda *s: torch.randn(*s, device=dev, generator=g, dtype=torch.float32)
    q = rms_norm(rn(B, H, T, D)).to(torch.bfloat16).requires_grad_(True)
    k = rms_norm(rn(B, H, T, D)).to(torch.bfloat16).requires_grad_(True)
    v = rn(B, H, T, D).to(torch.bfloat16).requires_grad_(True)
    do = rn(B, H, T, D).to(torch.bfloat16)
    sink = (rn(1, H, 1, 1) * 0.1).requires_grad_(True)
    N, d, V = HEAD["N"], HEAD["d"], HEAD["V"]
    h = rms_norm(rn(N, d)).to(torch.bfloat16).requires_grad_(True)
    E = (rn(V, d) * 0.02).to(torch.bfloat16).requires_grad_(True)
    t = torch.randint(0, V, (N,), device=dev, generator=g, dtype=torch.int32)
    return dict(q=q, k=k, v=v, do=do, sink=sink, h=h, E=E, t=t)


def make_steps(torch, x):
    from algebraic_amd.kernels.flash import flash_attention
    from algebraic_amd.kernels.fused_head import fused_head

    def attn_step():
        o = flash_attention(x["q"], x["k"], x["v"], x["sink"], kind="asinh", n=ATTN["n"], c=ATTN["c"],
                            block=512, range_guard=True)
        return torch.autograd.grad(o, (x["q"], x["k"], x["v"], x["sink"]), x["do"])

    def head_step():
        obj, _ = fused_head(x["h"], x["E"], x["t"], kind="alg_ce", n=HEAD["n"], c=HEAD["c"])
        return torch.autograd.grad(obj, (x["h"], x["E"]))

    def full_step():
        attn_step()
        head_step()

    return attn_step, head_step, full_step


def make_attn_step(torch, dev, B, H, T, D, seed=1):
    """Guarded bf16 attention fwd+bwd at another shape, inputs drawn as in make_inputs."""
    from algebraic_amd.kernels.flash import flash_attention
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    rn = lambda *s: torch.randn(*s, device=dev, generator=g, dtype=torch.float32)
    q = rms_norm(rn(B, H, T, D)).to(torch.bfloat16).requires_grad_(True)
    k = rms_norm(rn(B, H, T, D)).to(torch.bfloat16).requires_grad_(True)
    v = rn(B, H, T, D).to(torch.bfloat16).requires_grad_(True)
    sink = (rn(1, H, 1, 1) * 0.1).requires_grad_(True)
    do = rn(B, H, T, D).to(torch.bfloat16)

    def step():
        o = flash_attention(q, k, v, sink, kind="asinh", n=ATTN["n"], c=ATTN["c"], block=512, range_guard=True)
        return torch.autograd.grad(o, (q, k, v, sink), do)

    return step


PEAK_FP32_TFLOPS = 157.3   # MI355X dense fp32 MFMA

# The other BASELINE.json configs, reported beside the headline (timed unit: the wrapper call).
OTHER_CONFIGS = {
    "C1": dict(part="attn", dtype="f32", backward=False, B=2, H=12, T=1024, D=64,
               workload="attention fwd fp32 B2 H12 T1024 D64 (125M shape)"),
    "C2": dict(part="head", N=8192, d=768, V=50257,
               workload="fused alg_ce head fwd+bwd N8192 d768 V50257 bf16 (125M shape)"),
    "C3": dict(part="attn", dtype="bf16", backward=True, B=8, H=16, T=2048, D=64,
               workload="attention fwd+bwd bf16 B8 H16 T2048 D64 (350M shape)"),
    "C5": dict(part="attn", dtype="bf16", backward=False, B=1, H=16, T=16384, D=128,
               workload="attention fwd bf16 B1 H16 T16384 D128 (long context)"),
}


def time_other_configs(torch, dev, iters=20, warmup=3, seed=1):
    """Wrapper-call time of each other BASELINE config, with the same input distributions as
    the headline: ``ms`` is the mean of ``iters`` calls back to back between two events (as
    the headline step is timed), ``ms_single_call_median`` the median of ``iters`` calls each
    between its own events (host launch work before the first kernel included)."""
    from algebraic_amd.kernels.flash import flash_attention
    from algebraic_amd.kernels.fused_head import fused_head
    res = {}
    for name, cfg in OTHER_CONFIGS.items():
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        rn = lambda *s: torch.randn(*s, device=dev, generator=g, dtype=torch.float32)
        if cfg["part"] == "attn":
            B, H, T, D = cfg["B"], cfg["H"], cfg["T"], cfg["D"]
            dt = torch.bfloat16 if cfg["dtype"] == "bf16" else torch.float32
            bwd = cfg["backward"]
            q = rms_norm(rn(B, H, T, D)).to(dt).requires_grad_(bwd)
            k = rms_norm(rn(B, H, T, D)).to(dt).requires_grad_(bwd)
            v = rn(B, H, T, D).to(dt).requires_grad_(bwd)
            sink = (rn(1, H, 1, 1) * 0.1).requires_grad_(bwd)
            do = rn(B, H, T, D).to(dt)

            def call():
                if not bwd:
                    with torch.no_grad():
                        flash_attention(q, k, v, sink, kind="asinh", n=16, c=8.0, block=512, range_guard=True)
                    return
                o = flash_attention(q, k, v, sink, kind="asinh", n=16, c=8.0, block=512, range_guard=True)
                torch.autograd.grad(o, (q, k, v, sink), do)
            flops = attn_flops(B, H, T, D) * (3.5 if bwd else 1.0)
            tokens = B * T
            peak = PEAK_BF16_TFLOPS if dt == torch.bfloat16 else PEAK_FP32_TFLOPS
        else:
            N, d, V = cfg["N"], cfg["d"], cfg["V"]
            h = rms_norm(rn(N, d)).to(torch.bfloat16).requires_grad_(True)
            E = (rn(V, d) * 0.02).to(torch.bfloat16).requires_grad_(True)
            t = torch.randint(0, V, (N,), device=dev, generator=g, dtype=torch.int32)

            def call():
                obj, _ = fused_head(h, E, t, kind="alg_ce", n=8, c=2.0)
                torch.autograd.grad(obj, (h, E))
            flops = head_flops(N, d, V)
            tokens = N
            peak = PEAK_BF16_TFLOPS
        for _ in range(warmup):
            call()
        torch.cuda.synchronize()
        times = []
        for _ in range(iters):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            call()
            e1.record()
            e1.synchronize()
            times.append(e0.elapsed_time(e1))
        single = sorted(times)[len(times) // 2]
        # Steady state as the headline step is timed: `iters` calls back to back between two
        # events, so the wrapper's host work overlaps the previous call's kernels.
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(iters):
            call()
        e1.record()
        e1.synchronize()
        ms = e0.elapsed_time(e1) / iters
        tf = flops / (ms * 1e-3) / 1e12
        res[name] = {"workload": cfg["workload"], "ms": round(ms, 4), "tflops": round(tf, 3),
                     "tokens_per_s": round(tokens / (ms * 1e-3), 1), "peak": peak,
                     "frac_peak": round(tf / peak, 4), "flops": flops,
                     "ms_single_call_median": round(single, 4)}
    torch.cuda.synchronize()
    return res


def time_prologue(torch, dev, iters=20, warmup=3, seed=2):
    """Fused attention prologue at the C4a shape, raw projections in the (B, T, H, D) layout:
    forward (norm + gain, rotation, q pre-scale, guard) and VJP, each timed with CUDA events
    over ``iters`` calls (median). Algorithmic bytes: forward reads q, k, v and writes q_s,
    k_r and the two 1/rms rows; the VJP reads q, k, the two cotangents and 1/rms and writes
    dq, dk. Both are HBM-bound streams."""
    from algebraic_amd import _lib as L
    lib = L.load()
    B, H, T, D = (ATTN[k] for k in "BHTD")
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    rn = lambda *s: torch.randn(*s, device=dev, generator=g, dtype=torch.float32)
    q, k, v = (rn(B, T, H, D).to(torch.bfloat16) for _ in range(3))
    dq_r, dk_r = (rn(B, H, T, D).to(torch.bfloat16) for _ in range(2))
    gq, gk = 1 + 0.1 * rn(D), 1 + 0.1 * rn(D)
    from algebraic_amd.kernels.prologue import cayley_table_geometric
    cs, sn = cayley_table_geometric(D, T, device=dev)
    sink = 0.1 * rn(H)
    q_s, k_r = torch.empty((B, H, T, D), dtype=torch.bfloat16, device=dev), torch.empty((B, H, T, D), dtype=torch.bfloat16, device=dev)
    tau_q, tau_k = torch.empty((B, H, T), device=dev), torch.empty((B, H, T), device=dev)
    sink_out, flag = torch.empty(H, device=dev), torch.empty(1, dtype=torch.int32, device=dev)
    dq, dk = torch.empty_like(q), torch.empty_like(k)
    dgq, dgk = torch.empty(D, device=dev), torch.empty(D, device=dev)
    nbytes = lib.alg_attn_prologue_workspace_size(B, H, T, D)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    st = L.stream_of(q)
    P = L.ptr

    def fwd():
        L.check(lib.alg_attn_qk_prologue(st, L.DTYPE_BF16, L.LAYOUT_BTHD, B, H, T, D, P(q), P(k), P(v), P(gq), P(gk),
                                          P(cs), P(sn), 1e-5, P(sink), H, ATTN["c"], ATTN["n"], 1, P(q_s), P(k_r),
                                          P(tau_q), P(tau_k), P(sink_out), P(flag), P(ws), nbytes), "prologue")

    def bwd():
        L.check(lib.alg_attn_qk_prologue_bwd(st, L.DTYPE_BF16, L.LAYOUT_BTHD, B, H, T, D, P(q), P(k), P(gq), P(gk),
                                              P(cs), P(sn), P(tau_q), P(tau_k), P(dq_r), P(dk_r), P(dq), P(dk),
                                              P(dgq), P(dgk), P(ws), nbytes), "prologue bwd")

    def median_ms(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(iters):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            e1.synchronize()
            ts.append(e0.elapsed_time(e1))
        return sorted(ts)[len(ts) // 2]

    elems = B * H * T * D
    fwd_bytes = 5 * elems * 2 + 2 * B * H * T * 4
    bwd_bytes = 6 * elems * 2 + 2 * B * H * T * 4
    f_ms, b_ms = median_ms(fwd), median_ms(bwd)
    fg, bg = fwd_bytes / (f_ms * 1e-3) / 1e9, bwd_bytes / (b_ms * 1e-3) / 1e9
    return {"workload": "fused QK norm + gain + Cayley rotation + q*alpha + guard, C4a shape, (B,T,H,D) input",
            "fwd_ms": round(f_ms, 4), "fwd_bytes": fwd_bytes, "fwd_gbs": round(fg, 1),
            "bwd_ms": round(b_ms, 4), "bwd_bytes": bwd_bytes, "bwd_gbs": round(bg, 1),
            "peak_gbs": PEAK_HBM_GBS, "fwd_frac": round(fg / PEAK_HBM_GBS, 4), "bwd_frac": round(bg / PEAK_HBM_GBS, 4)}


def time_layout_bthd(torch, x, steps, warmup):
    """The headline attention step with q, k, v, dO stored (B, T, H, D) (the projection
    layout; o comes back as the (B, T, H*D) input of the output projection with no copy)."""
    from algebraic_amd.kernels.flash import flash_attention
    t = lambda a: a.detach().permute(0, 2, 1, 3).contiguous()
    q, k, v = (t(x[n]).requires_grad_(True) for n in ("q", "k", "v"))
    do = t(x["do"])

    def step():
        o = flash_attention(q, k, v, x["sink"], kind="asinh", n=ATTN["n"], c=ATTN["c"], block=512,
                            range_guard=True, layout="bthd")
        return torch.autograd.grad(o, (q, k, v, x["sink"]), do)
    s = timed(torch, step, steps, warmup)
    fa = attn_flops(**ATTN) * 3.5
    return {"workload": "C4a attention fwd+bwd with q, k, v, o, dO, dq, dk, dv in (B, T, H, D)",
            "ms": round(s * 1e3, 4), "tflops": round(fa / s / 1e12, 3)}


def kernel_times(torch, fn, iters):
    """Mean duration (ms) of each library kernel over `iters` calls of fn, from the library's
    HIP events on the launch stream (no host launch overhead)."""
    from algebraic_amd import _lib
    fn()
    torch.cuda.synchronize()
    _lib.timer_enable(True)
    for _ in range(iters):
        fn()
    torch.cuda.synchronize()
    rep = _lib.timer_report()
    _lib.timer_enable(False)
    return {name: r["mean_ms"] for name, r in rep.items()}


def time_eval_head(torch, x, iters=20, warmup=3):
    """Streamed evaluation head (per-token log p(target) and argmax, no logits) at the C4b
    shape; one N x d x V product, so TFLOP/s counts 2 N d V."""
    from algebraic_amd.kernels.fused_head import head_logprob
    h, E, t = x["h"].detach(), x["E"].detach(), x["t"]

    def call():
        head_logprob(h, E, t, n=HEAD["n"], c=HEAD["c"])
    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    ts = []
    for _ in range(iters):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        call()
        e1.record()
        e1.synchronize()
        ts.append(e0.elapsed_time(e1))
    ms = sorted(ts)[len(ts) // 2]
    k = kernel_times(torch, call, iters)
    fl = 2.0 * HEAD["N"] * HEAD["d"] * HEAD["V"]
    return {"workload": "eval head log p(target) + argmax, N16384 d2048 V32000 (C4b shape)",
            "ms": round(ms, 4), "tflops": round(fl / (ms * 1e-3) / 1e12, 3),
            "tokens_per_s": round(HEAD["N"] / (ms * 1e-3), 1),
            "kernel_ms": round(k["head_eval"], 4), "kernel_tflops": round(fl / (k["head_eval"] * 1e-3) / 1e12, 3),
            "stats_ms": round(k["head_eval_stats"], 4)}


def time_head_schedules(torch, x, iters=10, warmup=2):
    """The head's three backward schedules at the C4b shape, fwd+bwd each: "residual" (the
    default: a bf16 (N, V) residual from the forward, 3 products), "recompute" (the logits
    recomputed into an (N, V) bf16 logit-gradient workspace, 4 products) and "streamed" (the
    logits recomputed one vocabulary chunk at a time, no (N, V) block). `peak_extra_bytes` is
    the device memory the call allocates beyond its inputs at its peak (torch's allocator
    statistics), `nv_block_bytes` the (N, V)-sized buffer the schedule keeps."""
    from algebraic_amd import _lib
    from algebraic_amd.kernels import fused_head as FH
    lib = _lib.load()
    h, E, t = (x[k].detach() for k in ("h", "E", "t"))
    h = h.clone().requires_grad_(True)
    E = E.clone().requires_grad_(True)
    N, d, V = HEAD["N"], HEAD["d"], HEAD["V"]

    def call():
        obj, _ = FH.fused_head(h, E, t, kind="alg_ce", n=HEAD["n"], c=HEAD["c"])
        return torch.autograd.grad(obj, (h, E))
    saved = FH.SCHEDULE, FH.VOCAB_CHUNK
    out = {"workload": "fused alg_ce head fwd+bwd N16384 d2048 V32000 (C4b shape) per backward schedule"}
    nv = {"residual": lib.alg_head_residual_size(N, d, V),
          "recompute": lib.alg_head_workspace_size(_lib.DTYPE_BF16, N, d, V, 1),
          "streamed": 0}
    try:
        for sched in FH.SCHEDULES:
            FH.SCHEDULE, FH.VOCAB_CHUNK = sched, 0
            for _ in range(warmup):
                call()
            torch.cuda.synchronize()
            base = torch.cuda.memory_allocated()
            torch.cuda.reset_peak_memory_stats()
            call()
            torch.cuda.synchronize()
            peak = torch.cuda.max_memory_allocated() - base
            ts = []
            for _ in range(iters):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                call()
                e1.record()
                e1.synchronize()
                ts.append(e0.elapsed_time(e1))
            ms = sorted(ts)[len(ts) // 2]
            out[sched] = {"ms": round(ms, 4), "tflops": round(head_flops(**HEAD) / (ms * 1e-3) / 1e12, 3),
                          "peak_extra_bytes": int(peak), "nv_block_bytes": int(nv[sched])}
        out["streamed"]["workspace_bytes"] = int(lib.alg_head_streamed_workspace_size(_lib.DTYPE_BF16, N, d, V, 0))
    finally:
        FH.SCHEDULE, FH.VOCAB_CHUNK = saved
    return out


def time_step_graph(torch, x, full_step, steps, eager_ms):
    """The headline step captured once in a HIP graph (torch.cuda.CUDAGraph) and replayed
    `steps` times back to back: the launch-overhead-free time of the same kernels (the library
    reads no device data on the host and records no memset, and the range guard branches on
    the device, so the whole step replays). Reported beside the headline, not as it."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            full_step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        full_step()
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        graph.replay()
    e1.record()
    e1.synchronize()
    ms = e0.elapsed_time(e1) / steps
    del graph
    torch.cuda.synchronize()
    return {"workload": "the headline step (same kernels and shapes) replayed from one captured HIP graph",
            "ms": round(ms, 4), "eager_ms": round(eager_ms, 4), "eager_over_graph": round(eager_ms / ms, 4)}


def time_final_norm(torch, x, iters=20, warmup=3):
    """Final RMS norm with gain ahead of the head (model.py:208) at the C4b shape (16384 rows of
    2048): forward reads x, writes y (+ 1/rms); the VJP reads x, dy, writes dx (+ gain partials)."""
    from algebraic_amd.kernels.norm import rms_norm
    h = x["h"].detach().clone().requires_grad_(True)
    g = torch.ones(HEAD["d"], device=h.device, requires_grad=True)
    dy = torch.randn_like(h)

    def median_ms(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(iters):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            e1.synchronize()
            ts.append(e0.elapsed_time(e1))
        return sorted(ts)[len(ts) // 2]
    f_ms = median_ms(lambda: rms_norm(h, g))
    fb_ms = median_ms(lambda: torch.autograd.grad(rms_norm(h, g), (h, g), dy))
    # Kernel durations: the wrapper times above also hold the autograd and allocation
    # overhead of a ~0.1 ms call.
    k = kernel_times(torch, lambda: torch.autograd.grad(rms_norm(h, g), (h, g), dy), iters)
    kf, kb, kr = (k[n] for n in ("rms_norm_fwd", "rms_norm_bwd", "rms_norm_gain_reduce"))
    nb = HEAD["N"] * HEAD["d"] * 2
    fg, bg = (2 * nb) / (kf * 1e-3) / 1e9, (3 * nb) / (kb * 1e-3) / 1e9
    return {"workload": "final RMS norm + gain, 16384 x 2048 bf16 (C4b head input)",
            "fwd_kernel_ms": round(kf, 4), "fwd_gbs": round(fg, 1), "fwd_frac": round(fg / PEAK_HBM_GBS, 4),
            "bwd_kernel_ms": round(kb, 4), "bwd_gbs": round(bg, 1), "bwd_frac": round(bg / PEAK_HBM_GBS, 4),
            "gain_reduce_ms": round(kr, 4), "wrapper_fwd_ms": round(f_ms, 4), "wrapper_fwd_bwd_ms": round(fb_ms, 4),
            "peak_gbs": PEAK_HBM_GBS}


def time_ffn(torch, dev, iters=10, warmup=2, seed=3):
    """ALU-GLU feed-forward at the 1b model's shape (N = 8 x 2048 tokens, d 1536, d_ff 4224):
    the fused gate/up product (2 N d 2F FLOP) and the fused dy product (2 N d F), the whole
    block forward + backward, and the same block with plain library products and torch
    elementwise activation for comparison."""
    from algebraic_amd import _lib as L
    from algebraic_amd.kernels.ffn import alu_glu_ffn
    N, d, F = 16384, 1536, 4224
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    rn = lambda *s, sc=1.0: (torch.randn(*s, device=dev, generator=g) * sc).to(torch.bfloat16)
    h2 = rn(N, d).requires_grad_(True)
    w_g, w_u = rn(d, F, sc=d ** -0.5).requires_grad_(True), rn(d, F, sc=d ** -0.5).requires_grad_(True)
    w_d = rn(F, d, sc=F ** -0.5).requires_grad_(True)
    dout = rn(N, d)

    def median_ms(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(iters):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            e1.synchronize()
            ts.append(e0.elapsed_time(e1))
        return sorted(ts)[len(ts) // 2]

    def fused():
        torch.autograd.grad(alu_glu_ffn(h2, w_g, w_u, w_d, 0.5), (h2, w_g, w_u, w_d), dout)

    def plain():
        up = h2 @ w_u
        act = (0.5 * up.float() * (1 + 0.5 * up.float() * torch.rsqrt(1 + (0.5 * up.float()) ** 2))).to(up.dtype)
        out = ((h2 @ w_g) * act) @ w_d
        torch.autograd.grad(out, (h2, w_g, w_u, w_d), dout)
    lib = L.load()
    w_gu = torch.cat([w_g, w_u], 1).detach().contiguous()
    y, gate, up = (torch.empty((N, F), dtype=torch.bfloat16, device=dev) for _ in range(3))
    d_gu = torch.empty((N, 2 * F), dtype=torch.bfloat16, device=dev)
    st = L.stream_of(h2)
    def both():
        L.check(lib.alg_ffn_alu_glu_fwd(st, N, d, F, L.ptr(h2), L.ptr(w_gu), 0.5, L.ptr(y), L.ptr(gate), L.ptr(up)),
                "ffn fwd")
        L.check(lib.alg_ffn_alu_glu_dy(st, N, d, F, L.ptr(dout), L.ptr(w_d.detach()), L.ptr(gate), L.ptr(up), 0.5,
                                       L.ptr(d_gu)), "ffn dy")
    k = kernel_times(torch, both, iters)
    k_fwd, k_dy = k["ffn_gate_up"], k["ffn_dy"]
    t_f, t_p = median_ms(fused), median_ms(plain)
    fl_gu, fl_dy = 2.0 * N * d * 2 * F, 2.0 * N * d * F
    block = 9 * 2.0 * N * d * F  # 3 products of 2 N d F forward (gate, up, out), 6 backward
    return {"workload": "ALU-GLU FFN, 1b shape N16384 d1536 d_ff4224 bf16",
            "gate_up_ms": round(k_fwd, 4), "gate_up_tflops": round(fl_gu / (k_fwd * 1e-3) / 1e12, 1),
            "dy_ms": round(k_dy, 4), "dy_tflops": round(fl_dy / (k_dy * 1e-3) / 1e12, 1),
            "block_fwd_bwd_ms": round(t_f, 4), "block_tflops": round(block / (t_f * 1e-3) / 1e12, 1),
            "plain_library_ms": round(t_p, 4), "vs_plain": round(t_p / t_f, 3)}


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` recorded from rocprofv3 FETCH_SIZE + WRITE_SIZE runs
    (each scaled by the same counter's reading for a device copy of known size), as listed
    in profiles/hbm_traffic_1b.txt; None when the kernel has no recorded figure."""
    path = ROOT / "profiles" / "hbm_traffic_1b.txt"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        fields = dict(f.split("=", 1) for f in line.split() if "=" in f)
        if fields.get("kernel") == kernel and "traffic_bytes" in fields:
            return int(float(fields["traffic_bytes"]))
    return None


def timed(torch, fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def _cpu_model():
    """The host CPU's model name (first processor in /proc/cpuinfo), or None."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def _median_time(fn, runs=3, warmup=1):
    """Median wall time of `runs` calls after `warmup` untimed ones, and every timed sample."""
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2], ts


def cpu_baseline(c1_gpu_ms=None):
    """The NumPy oracle (float32, the cast-faithful restatement of the reference's algorithm)
    timed on the host cores: one warmup and the median of three runs each of a bounded sample
    of the step (attention fwd+bwd on a few heads, head fwd+bwd on a few tokens, scaled to the
    full step) and of BASELINE config 1 (attention forward, fp32, B2 H12 T1024 D64) at full
    shape. BLAS threads: the affinity mask's cores, capped at OMP_NUM_THREADS when the host
    sets it (a GPU box's share of the host)."""
    import numpy as np
    from oracle import attention as OA
    from oracle import head as OH
    from oracle.numerics import round_bf16
    from threadpoolctl import threadpool_info, threadpool_limits
    affinity = len(os.sched_getaffinity(0))
    threads = min(affinity, int(os.environ.get("OMP_NUM_THREADS") or affinity))
    rng = np.random.default_rng(0)
    B, H, T, D = (ATTN[k] for k in "BHTD")
    nh = 4
    mk = lambda: round_bf16(rng.standard_normal((1, nh, T, D)).astype(np.float32))
    q, k, v, do = mk(), mk(), mk(), mk()
    sink = (rng.standard_normal((1, nh, 1, 1)) * 0.1).astype(np.float32)
    N, d, V = HEAD["N"], HEAD["d"], HEAD["V"]
    ns = (128, 384)  # two token counts: per-call work (E's cast, dE's rounding) is not per token
    h = round_bf16(rng.standard_normal((ns[1], d)).astype(np.float32))
    E = round_bf16((rng.standard_normal((V, d)) * 0.02).astype(np.float32))
    tg = rng.integers(0, V, ns[1])
    c1 = OTHER_CONFIGS["C1"]
    c1x = [rng.standard_normal((c1["B"], c1["H"], c1["T"], c1["D"])).astype(np.float32) for _ in range(3)]
    c1s = (rng.standard_normal((1, c1["H"], 1, 1)) * 0.1).astype(np.float32)

    def attn_sample():
        OA.flash_attention_oracle(q, k, v, sink, do, n=ATTN["n"], c=ATTN["c"], dtype="bf16")

    def head_sample(m):
        stat, _, _, _ = OH.kernel_forward(h[:m], E, tg[:m], n=HEAD["n"], c=HEAD["c"], chunk=128)
        OH.kernel_backward(h[:m], E, tg[:m], stat, 1.0, n=HEAD["n"], c=HEAD["c"], chunk=128)

    def c1_forward():
        OA.flash_attention_oracle(*c1x, c1s, n=ATTN["n"], c=ATTN["c"], dtype="f32")

    with threadpool_limits(limits=threads):
        blas = max([p.get("num_threads", 1) for p in threadpool_info()] or [1])
        ta, ta_runs = _median_time(attn_sample)
        th0, th0_runs = _median_time(lambda: head_sample(ns[0]))
        th1, th1_runs = _median_time(lambda: head_sample(ns[1]), warmup=0)
        tc1, tc1_runs = _median_time(c1_forward)
    t_attn = ta / nh * (B * H)
    per_token = max(th1 - th0, 0.0) / (ns[1] - ns[0])
    t_head = th0 + per_token * (N - ns[0])  # the per-call part once, the per-token part N times
    total = attn_flops(**ATTN) * 3.5 + head_flops(**HEAD)
    step_s = t_attn + t_head
    c1_flops = attn_flops(**c1)
    out = {
        "value": round(total / step_s / 1e12, 6), "unit": "TFLOP/s", "cores": int(blas), "kind": "port",
        "sample": (f"NumPy float32 oracle (oracle/attention.py kernel_forward/backward, oracle/head.py "
                   f"kernel_forward/backward), one warmup then the median of 3 runs: attention fwd+bwd on "
                   f"{nh} of {B * H} heads (T={T}, D={D}) scaled x{B * H // nh}, head fwd+bwd on {ns[0]} and "
                   f"{ns[1]} of {N} tokens (d={d}, V={V}) extrapolated linearly to {N} tokens; est. CPU "
                   f"step {step_s:.1f} s (attention {t_attn:.1f} s, head {t_head:.1f} s)"),
        "cpu_model": _cpu_model(),
        "affinity_cores": affinity,
        "blas_threads": int(blas),
        "runs_s": {"attention_sample": [round(x, 4) for x in ta_runs],
                   f"head_sample_{ns[0]}": [round(x, 4) for x in th0_runs],
                   f"head_sample_{ns[1]}": [round(x, 4) for x in th1_runs]},
        "C1": {"workload": c1["workload"] + ", full shape", "ms": round(tc1 * 1e3, 3),
               "tflops": round(c1_flops / tc1 / 1e12, 6), "runs_ms": [round(x * 1e3, 3) for x in tc1_runs]},
    }
    if c1_gpu_ms:
        out["C1"]["gpu_ms"] = c1_gpu_ms
        out["C1"]["gpu_speedup"] = round(tc1 * 1e3 / c1_gpu_ms, 1)
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip timing BASELINE configs 1, 2, 3 and 5 beside the headline")
    ap.add_argument("--only", choices=["attn", "head", "step", "neighbours", "c3", "head_schedules"],
                    help="run only W+K launches of one part (for profiler runs) and print its time; "
                         "'c3' is the attention fwd+bwd of BASELINE config 3 (D = 64); "
                         "'neighbours' runs the timings of the fused prologue, eval head, final norm "
                         "and feed-forward")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="with --only: also run K device copies of this many MiB (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build measures one MI355X "
              "(the path shards over (batch, head) and token blocks without cross-GPU exchange; "
              "one GPU share is the kernel at its real shape). Run with --gpus 1.", file=sys.stderr)
        return 2
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    from algebraic_amd import _lib
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    x = make_inputs(torch, dev)
    attn_step, head_step, full_step = make_steps(torch, x)

    K, W = args.steps, args.warmup
    log = lambda msg: print(f"bench: {msg}", file=sys.stderr, flush=True)
    if args.only == "head_schedules":
        print(json.dumps({"only": "head_schedules", **time_head_schedules(torch, x, iters=K, warmup=W)}), flush=True)
        return 0
    if args.only == "neighbours":
        out = {"only": "neighbours", "prologue": time_prologue(torch, dev), "eval_head": time_eval_head(torch, x),
               "final_norm": time_final_norm(torch, x), "ffn": time_ffn(torch, dev)}
        print(json.dumps(out), flush=True)
        return 0
    if args.only:
        if args.only == "c3":
            attn_step = make_attn_step(torch, dev, **{k: OTHER_CONFIGS["C3"][k] for k in "BHTD"})
        fn = {"attn": attn_step, "c3": attn_step, "head": head_step, "step": full_step}[args.only]
        t = timed(torch, fn, K, W)
        res = {"only": args.only, "steps": K, "warmup": W, "ms": round(t * 1e3, 4)}
        if args.copy_mib:
            nbytes = args.copy_mib << 20
            src = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1)
            dst = torch.empty_like(src)
            for _ in range(K):
                dst.copy_(src)
            torch.cuda.synchronize()
            res["copy_bytes"] = nbytes
        print(json.dumps(res), flush=True)
        return 0
    step_s = timed(torch, full_step, K, W)
    log(f"full step {step_s * 1e3:.3f} ms")
    attn_s = timed(torch, attn_step, K, 1)
    log(f"attention fwd+bwd {attn_s * 1e3:.3f} ms")
    head_s = timed(torch, head_step, K, 1)
    log(f"head fwd+bwd {head_s * 1e3:.3f} ms")

    # Per-kernel durations from HIP events on the launch stream (separate timed pass).
    _lib.timer_enable(True)
    for _ in range(K):
        full_step()
    torch.cuda.synchronize()
    kernels = _lib.timer_report()
    _lib.timer_enable(False)

    fa = attn_flops(**ATTN) * 3.5
    fh = head_flops(**HEAD)
    attn_tf = fa / attn_s / 1e12
    head_tf = fh / head_s / 1e12
    algo = kernel_algorithmic_flops()
    per_step = {name: rec["mean_ms"] * rec["launches"] / K for name, rec in kernels.items()}
    dom = max(per_step, key=per_step.get)
    dom_ms = kernels[dom]["mean_ms"]
    achieved = algo.get(dom, 0.0) / (dom_ms * 1e-3) / 1e12 if dom in algo else None

    def in_step(prefix, flops):
        """A part's time inside the full step: the sum of its kernels' HIP-event durations
        in the timed step pass (the standalone loop above runs the part alone, back to back)."""
        ms = sum(v for n, v in per_step.items() if n.startswith(prefix))
        tf = flops / (ms * 1e-3) / 1e12
        return {"in_step_kernels_ms": round(ms, 4), "in_step_tflops": round(tf, 3),
                "in_step_frac_peak": round(tf / PEAK_BF16_TFLOPS, 4)}
    roofline = {
        "kernel": dom,
        "bound": "mfma",
        "achieved": round(achieved, 3) if achieved is not None else None,
        "peak": PEAK_BF16_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(achieved / PEAK_BF16_TFLOPS, 4) if achieved is not None else None,
        "traffic": measured_traffic(dom),
        "mean_ms": round(dom_ms, 4),
    }
    out = {
        "metric": METRIC,
        "value": round((fa + fh) / step_s / 1e12, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(step_s * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": ("1B shape (BASELINE config 4): causal algebraic attention fwd+bwd "
                         "B8 H16 T2048 D128 n16 c8 range_guard + fused alg_ce head fwd+bwd "
                         "N16384 d2048 V32000 n8 c2"),
            "tokens_per_step": HEAD["N"],
            "flops_per_step": fa + fh,
        },
        "attn": {
            "ms": round(attn_s * 1e3, 4), "tflops": round(attn_tf, 3),
            "tokens_per_s": round(ATTN["B"] * ATTN["T"] / attn_s, 1),
            "frac_peak": round(attn_tf / PEAK_BF16_TFLOPS, 4),
            **in_step("attn_", fa),
        },
        "head": {
            "ms": round(head_s * 1e3, 4), "tflops": round(head_tf, 3),
            "tokens_per_s": round(HEAD["N"] / head_s, 1),
            "frac_peak": round(head_tf / PEAK_BF16_TFLOPS, 4),
            **in_step("head_", fh),
        },
        "kernels": {n: {"launches_per_step": r["launches"] / K, "mean_ms": round(r["mean_ms"], 4),
                        **({"tflops": round(algo[n] / (r["mean_ms"] * 1e-3) / 1e12, 2)} if n in algo else {})}
                    for n, r in sorted(kernels.items())},
        "roofline": roofline,
    }
    if not args.no_other_configs:
        log("timing the other BASELINE configs (C1, C2, C3, C5)")
        out["other_configs"] = time_other_configs(torch, dev)
        out["prologue"] = time_prologue(torch, dev)
        out["layout_bthd"] = time_layout_bthd(torch, x, K, 1)
        out["layout_bthd"]["vs_bhtd"] = round(out["attn"]["ms"] / out["layout_bthd"]["ms"], 4)
        out["eval_head"] = time_eval_head(torch, x)
        out["head_schedules"] = time_head_schedules(torch, x)
        out["final_norm"] = time_final_norm(torch, x)
        out["ffn"] = time_ffn(torch, dev)
        out["step_graph"] = time_step_graph(torch, x, full_step, K, step_s * 1e3)
    if not args.no_cpu_baseline:
        log("timing the CPU baseline sample")
        c1_ms = out.get("other_configs", {}).get("C1", {}).get("ms")
        out["cpu_baseline"] = cpu_baseline(c1_ms)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
