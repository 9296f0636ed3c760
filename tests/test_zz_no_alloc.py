"""GPU check of alg_attn_bwd_noalloc, the allocation-free attention backward.

It has no counterpart in the reference; it serves callers that cannot allocate device memory.
Through the C ABI (ctypes), each call is checked against alg_attn_bwd with a caller workspace
on the same forward residuals, for two calls in a row, the second with a smaller input (the
scratch keeps the first call's contents): bf16 results bit-identical (the same kernels, no
atomics); f32 dk, dv, di and dsink bit-identical and dq within 1e-6 (it is added with f32
atomics, whose order varies). The device's free memory (hipMemGetInfo) is the same before
and after each checked call.
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


def _outputs(k, v):
    B, H, T, D = k.shape
    return [torch.empty_like(k), torch.empty_like(k), torch.empty_like(v),
            torch.empty((B, H, T), dtype=torch.float32, device="cuda"), torch.empty(H, dtype=torch.float32, device="cuda")]


def _backward(r, k, v, do, noalloc, out=None):
    """One backward through the C ABI into `out` (allocated here if not given). For the
    no-alloc entry point the device's free memory (hipMemGetInfo) is read before the call and
    after it has finished; the difference is returned with the results."""
    L = _lib()
    lib = L.load()
    B, H, T, D = k.shape
    st = L.stream_of(k)
    dq, dk, dv, di, dsink = out if out is not None else _outputs(k, v)
    args = [st, r["dt"], 0, B, H, T, D, L.ptr(r["q_s"]), L.ptr(k), L.ptr(v), L.ptr(r["sink_s"]), L.ptr(r["o"]),
            L.ptr(r["stat"]), L.ptr(do), r["n"], L.ATTN_GUARDED, L.ptr(r["flag"]), r["clamp"], 1, 1, r["alpha"],
            L.ptr(dq), L.ptr(dk), L.ptr(dv), L.ptr(di), L.ptr(dsink)]
    freed = 0
    if noalloc:
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        L.check(lib.alg_attn_bwd_noalloc(*args), "alg_attn_bwd_noalloc")
        torch.cuda.synchronize()
        freed = free0 - torch.cuda.mem_get_info()[0]
    else:
        ws_bytes = lib.alg_attn_workspace_size(r["dt"], B, H, T, D)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
        L.check(lib.alg_attn_bwd(*args, L.ptr(ws), ws_bytes), "alg_attn_bwd")
    torch.cuda.synchronize()
    return [x.float().cpu().numpy() for x in (dq, dk, dv, di, dsink)], freed


@pytest.mark.parametrize("dtype,shapes", [
    (torch.bfloat16, [(2, 4, 384, 128), (1, 2, 200, 64)]),
    (torch.float32, [(1, 3, 512, 64), (1, 2, 100, 64)]),
])
def test_noalloc_backward_matches_the_workspace_entry_point(dtype, shapes):
    """Both calls match the workspace entry point, and neither changes the device's free
    memory: everything the calls need (inputs, outputs, the library's code and its static
    scratch array) exists before them. A first call on a smaller shape sets up the scratch
    address (hipGetSymbolAddress, once per device) before the calls that are checked."""
    cases = []
    for call, (B, H, T, D) in enumerate(shapes):
        q, k, v, do, sink = attention_inputs(B, H, T, D, seed=40 + call, dtype="bf16" if dtype == torch.bfloat16
                                             else "f32")
        tq, tk, tv, tdo = (torch.tensor(a, device="cuda").to(dtype) for a in (q, k, v, do))
        tsink = torch.tensor(sink.reshape(-1), device="cuda")
        res = _forward(tq, tk, tv, tsink, dtype)
        want = _backward(res, tk, tv, tdo, noalloc=False)[0]
        cases.append((res, tk, tv, tdo, want, _outputs(tk, tv)))
    res, tk, tv, tdo, _, out = cases[-1]
    _backward(res, tk, tv, tdo, noalloc=True, out=out)  # set-up call
    for call, (res, tk, tv, tdo, want, out) in enumerate(cases):
        print(f"[noalloc] call {call}: {dtype} {tuple(tk.shape)}", flush=True)
        got, freed = _backward(res, tk, tv, tdo, noalloc=True, out=out)
        assert freed == 0, f"call {call}: device free memory fell by {freed} bytes"
        names = ("dq", "dk", "dv", "di", "dsink")
        for name, a, b in zip(names, got, want):
            if dtype == torch.float32 and name == "dq":
                np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-9, err_msg=name)
            else:
                np.testing.assert_array_equal(a, b, err_msg=name)
