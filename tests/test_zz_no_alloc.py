"""GPU check of alg_attn_bwd_noalloc, the allocation-free attention backward.

It has no counterpart in the reference; it serves callers that cannot allocate device memory.
Through the C ABI (ctypes), each call is checked against alg_attn_bwd with a caller workspace
on the same forward residuals, for two calls in a row, the second with a smaller input (the
scratch keeps the first call's contents): bf16 results bit-identical (the same kernels, no
atomics); f32 dk, dv, di and dsink bit-identical and dq within 1e-6 (it is added with f32
atomics, whose order varies).
"""

import ctypes
import math

import numpy as np
import pytest

from helpers import attention_inputs

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _lib():
    from algebraic_amd import _lib
    return _lib


def _forward(q, k, v, sink, dtype, n=16, c=8.0):
    """Guarded prologue + forward through the C ABI; returns the backward's residuals."""
    L = _lib()
    lib = L.load()
    B, H, T, D = q.shape
    dt = L.DTYPE_BF16 if dtype == torch.bfloat16 else L.DTYPE_F32
    st = L.stream_of(q)
    ws_bytes = lib.alg_attn_workspace_size(dt, B, H, T, D)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    q_s = torch.empty_like(q)
    sink_s = torch.empty(H, dtype=torch.float32, device="cuda")
    flag = torch.empty(1, dtype=torch.int32, device="cuda")
    L.check(lib.alg_attn_prepare(st, dt, B, H, T, D, L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(sink), H, c, n, 1,
                                 L.ptr(q_s), L.ptr(sink_s), L.ptr(flag), L.ptr(ws), ws_bytes), "prepare")
    o = torch.empty_like(q)
    stat = torch.empty((B, H, T), dtype=torch.float32, device="cuda")
    t = 1e37 / (T + 1.0)
    for _ in range(4):
        t = math.sqrt(t)
    clamp = 0.5 * (t - 1.0 / t)
    L.check(lib.alg_attn_fwd(st, dt, 0, B, H, T, D, L.ptr(q_s), L.ptr(k), L.ptr(v), L.ptr(sink_s), n,
                             L.ATTN_GUARDED, L.ptr(flag), clamp, 1, 1, L.ptr(o), None, L.ptr(stat)), "forward")
    return dict(dt=dt, q_s=q_s, sink_s=sink_s, flag=flag, o=o, stat=stat, clamp=clamp, n=n,
                alpha=1.0 / (math.sqrt(D) * c))


def _backward(r, k, v, do, noalloc):
    L = _lib()
    lib = L.load()
    B, H, T, D = k.shape
    st = L.stream_of(k)
    dq, dk, dv = torch.empty_like(k), torch.empty_like(k), torch.empty_like(v)
    di = torch.empty((B, H, T), dtype=torch.float32, device="cuda")
    dsink = torch.empty(H, dtype=torch.float32, device="cuda")
    args = [st, r["dt"], 0, B, H, T, D, L.ptr(r["q_s"]), L.ptr(k), L.ptr(v), L.ptr(r["sink_s"]), L.ptr(r["o"]),
            L.ptr(r["stat"]), L.ptr(do), r["n"], L.ATTN_GUARDED, L.ptr(r["flag"]), r["clamp"], 1, 1, r["alpha"],
            L.ptr(dq), L.ptr(dk), L.ptr(dv), L.ptr(di), L.ptr(dsink)]
    if noalloc:
        L.check(lib.alg_attn_bwd_noalloc(*args), "alg_attn_bwd_noalloc")
    else:
        ws_bytes = lib.alg_attn_workspace_size(r["dt"], B, H, T, D)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
        L.check(lib.alg_attn_bwd(*args, L.ptr(ws), ws_bytes), "alg_attn_bwd")
    torch.cuda.synchronize()
    return [x.float().cpu().numpy() for x in (dq, dk, dv, di, dsink)]


@pytest.mark.parametrize("dtype,shapes", [
    (torch.bfloat16, [(2, 4, 384, 128), (1, 2, 200, 64)]),
    (torch.float32, [(1, 3, 512, 64), (1, 2, 100, 64)]),
])
def test_noalloc_backward_matches_the_workspace_entry_point(dtype, shapes):
    for call, (B, H, T, D) in enumerate(shapes):
        print(f"[noalloc] call {call}: {dtype} B{B} H{H} T{T} D{D}", flush=True)
        q, k, v, do, sink = attention_inputs(B, H, T, D, seed=40 + call, dtype="bf16" if dtype == torch.bfloat16
                                             else "f32")
        tq, tk, tv, tdo = (torch.tensor(a, device="cuda").to(dtype) for a in (q, k, v, do))
        tsink = torch.tensor(sink.reshape(-1), device="cuda")
        res = _forward(tq, tk, tv, tsink, dtype)
        want = _backward(res, tk, tv, tdo, noalloc=False)
        got = _backward(res, tk, tv, tdo, noalloc=True)
        names = ("dq", "dk", "dv", "di", "dsink")
        for name, a, b in zip(names, got, want):
            if dtype == torch.float32 and name == "dq":
                np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-9, err_msg=name)
            else:
                np.testing.assert_array_equal(a, b, err_msg=name)
