"""The hot path captured in a HIP graph (torch.cuda.CUDAGraph) and replayed.

The step is what bench.py times, through the drop-in mirrors: guarded causal attention forward
and backward (flash_attention(range_guard=True), flash.py:763-857 with its VJP) and the fused
head forward and backward (fused_head, fused_head.py:232-275). None of the library's calls
reads device data on the host, allocates, or records a memset, so the whole sequence can be
captured once and replayed. The range guard is decided on the device (the guard kernel writes
a flag that the in-range and fallback kernels read), so one captured graph takes whichever
branch the replayed inputs need: the third case below has a key row that fails the guard
(||q_s||^2 ||k||^2 above (16/1.01)^2, flash.py:834-849), and its replay runs the shifted
fallback. Each replay follows eager work (new inputs copied in) and a synchronisation, and
every output of every replay is compared with an eager run of the same step on the same
inputs: bit-identical (the kernels are deterministic and the replay launches the same kernels
with the same shapes).
"""

import math

import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

B, H, T, D = 2, 4, 512, 128
N, DM, V = 512, 256, 3000
N_EXP, C = 16, 8.0


def _rms(x):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)


def _case(seed, big_key=False):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    rn = lambda *s: torch.randn(*s, device="cuda", generator=g, dtype=torch.float32)
    k = _rms(rn(B, H, T, D))
    if big_key:
        k[1, 2, 300] *= 12.0  # ||k||^2 = 144 D: the guard's product 144 D^2 alpha^2 > (16/1.01)^2
    return dict(q=_rms(rn(B, H, T, D)).to(torch.bfloat16), k=k.to(torch.bfloat16),
                v=rn(B, H, T, D).to(torch.bfloat16), sink=rn(1, H, 1, 1) * 0.1,
                do=rn(B, H, T, D).to(torch.bfloat16), h=_rms(rn(N, DM)).to(torch.bfloat16),
                E=(rn(V, DM) * 0.02).to(torch.bfloat16),
                t=torch.randint(0, V, (N,), device="cuda", generator=g, dtype=torch.int32))


def _guard_flag(x):
    """The guard's decision for inputs x, from one eager alg_attn_fwd_guarded call (1: in range)."""
    from algebraic_amd import _lib as L
    lib = L.load()
    dt = L.DTYPE_BF16
    ws_bytes = lib.alg_attn_workspace_size(dt, B, H, T, D)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    sink_in = x["sink"].reshape(-1).contiguous()
    q_s, o = torch.empty_like(x["q"]), torch.empty_like(x["q"])
    sink_s = torch.empty(H, dtype=torch.float32, device="cuda")
    flag = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    stat = torch.empty((B, H, T), dtype=torch.float32, device="cuda")
    L.check(lib.alg_attn_fwd_guarded(L.stream_of(x["q"]), dt, 0, B, H, T, D, L.ptr(x["q"]), L.ptr(x["k"]),
                                     L.ptr(x["v"]), L.ptr(sink_in), H, C, N_EXP, L.ptr(q_s), L.ptr(sink_s),
                                     L.ptr(flag), L.ptr(o), None, L.ptr(stat), L.ptr(ws), ws_bytes), "guarded")
    torch.cuda.synchronize()
    return int(flag.item())


def test_step_graph_replays_match_eager():
    from algebraic_amd.kernels.flash import flash_attention
    from algebraic_amd.kernels.fused_head import fused_head

    first = _case(1)
    q, k, v, do = (first[n].clone().requires_grad_(n != "do") for n in ("q", "k", "v", "do"))
    sink = first["sink"].clone().requires_grad_(True)
    h, E = first["h"].clone().requires_grad_(True), first["E"].clone().requires_grad_(True)
    t = first["t"].clone()

    def step():
        o = flash_attention(q, k, v, sink, kind="asinh", n=N_EXP, c=C, block=512, range_guard=True)
        dq, dk, dv, ds = torch.autograd.grad(o, (q, k, v, sink), do)
        obj, tel = fused_head(h, E, t, kind="alg_ce", n=8, c=2.0)
        dh, dE = torch.autograd.grad(obj, (h, E))
        return o, dq, dk, dv, ds, obj, tel, dh, dE

    names = ("o", "dq", "dk", "dv", "dsink", "obj", "tel", "dh", "dE")
    # Warm-up on a side stream before capture (torch's capture recipe), then one capture.
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = step()
    torch.cuda.synchronize()

    cases = [("in range, capture inputs", first), ("in range, new inputs", _case(2)),
             ("guard fails on one key row", _case(3, big_key=True))]
    assert _guard_flag(cases[1][1]) == 1 and _guard_flag(cases[2][1]) == 0, "case inputs"
    for label, x in cases:
        print(f"[graph] replay: {label}", flush=True)
        with torch.no_grad():
            for dst, n in ((q, "q"), (k, "k"), (v, "v"), (do, "do"), (sink, "sink"), (h, "h"), (E, "E"), (t, "t")):
                dst.copy_(x[n])
        want = [w.detach().clone() for w in step()]  # eager, same inputs
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, got, ref in zip(names, static_out, want):
            assert torch.isfinite(ref.float()).all(), (label, name)
            assert torch.equal(got, ref), (label, name, (got.float() - ref.float()).abs().max().item())
    # The replay after the failing case again takes the in-range branch.
    with torch.no_grad():
        for dst, n in ((q, "q"), (k, "k"), (v, "v"), (do, "do"), (sink, "sink"), (h, "h"), (E, "E"), (t, "t")):
            dst.copy_(first[n])
    want = [w.detach().clone() for w in step()]
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    for name, got, ref in zip(names, static_out, want):
        assert torch.equal(got, ref), ("back in range", name)
    assert not math.isnan(float(static_out[5].item()))


def test_noalloc_backward_in_a_graph():
    """alg_attn_bwd_noalloc (no counterpart in the reference; for callers that cannot allocate,
    such as code under graph capture) captured in a graph through the C ABI and replayed for
    three upstream gradients: every replay bit-identical (bf16) to the workspace entry point
    alg_attn_bwd run eagerly on the same inputs. One eager call first sets up the library's
    scratch address (once per device, outside the capture)."""
    from algebraic_amd import _lib as L
    lib = L.load()
    Bb, Hb, Tb, Db = 2, 4, 384, 128
    dt = L.DTYPE_BF16
    x = _case(4)
    q, k, v = (x[n][:Bb, :Hb, :Tb].contiguous() for n in ("q", "k", "v"))
    sink_in = x["sink"][:, :Hb].reshape(-1).contiguous()
    st = L.stream_of(q)
    ws_bytes = lib.alg_attn_workspace_size(dt, Bb, Hb, Tb, Db)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    q_s, o = torch.empty_like(q), torch.empty_like(q)
    sink_s = torch.empty(Hb, dtype=torch.float32, device="cuda")
    flag = torch.empty(1, dtype=torch.int32, device="cuda")
    stat = torch.empty((Bb, Hb, Tb), dtype=torch.float32, device="cuda")
    L.check(lib.alg_attn_fwd_guarded(st, dt, 0, Bb, Hb, Tb, Db, L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(sink_in), Hb,
                                     C, N_EXP, L.ptr(q_s), L.ptr(sink_s), L.ptr(flag), L.ptr(o), None, L.ptr(stat),
                                     L.ptr(ws), ws_bytes), "guarded forward")
    t = 1e37 / (Tb + 1.0)
    for _ in range(4):
        t = math.sqrt(t)
    clamp, alpha = 0.5 * (t - 1.0 / t), 1.0 / (math.sqrt(Db) * C)
    do = torch.empty_like(q)

    def outputs():
        return [torch.empty_like(k), torch.empty_like(k), torch.empty_like(v),
                torch.empty((Bb, Hb, Tb), dtype=torch.float32, device="cuda"),
                torch.empty(Hb, dtype=torch.float32, device="cuda")]

    def args(out, stream):
        return [stream, dt, 0, Bb, Hb, Tb, Db, L.ptr(q_s), L.ptr(k), L.ptr(v), L.ptr(sink_s), L.ptr(o), L.ptr(stat),
                L.ptr(do), N_EXP, L.ATTN_GUARDED, L.ptr(flag), clamp, 1, 1, alpha, *(L.ptr(a) for a in out)]

    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    do.copy_(torch.randn(do.shape, device="cuda", generator=g).to(torch.bfloat16))
    static = outputs()
    L.check(lib.alg_attn_bwd_noalloc(*args(static, st)), "set-up call")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        L.check(lib.alg_attn_bwd_noalloc(*args(static, L.stream_of(q))), "captured call")
    torch.cuda.synchronize()
    for rep in range(3):
        print(f"[graph] no-alloc backward replay {rep}", flush=True)
        do.copy_(torch.randn(do.shape, device="cuda", generator=g).to(torch.bfloat16))
        want = outputs()
        L.check(lib.alg_attn_bwd(*args(want, st), L.ptr(ws), ws_bytes), "eager workspace backward")
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("dq", "dk", "dv", "di", "dsink"), static, want):
            assert torch.isfinite(b.float()).all(), (rep, name)
            assert torch.equal(a, b), (rep, name)
