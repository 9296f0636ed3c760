"""GPU check of alg_attn_fwd_guarded, the guarded forward from unscaled queries in one call.

For bf16 inputs, and f32 at D = 64, the in-range forward kernel forms q * alpha itself, writes
q_s and leaves the guard maxima of its rows; the guard runs after it and the flag-checked shifted branch
replaces o and stat when the guard fails (flash.py:823-856). Through the C ABI (ctypes) every
output is compared with the two-call sequence alg_attn_prepare(range_guard=1) +
alg_attn_fwd(GUARDED) on the same inputs: q_s, sink/c, the flag, o and stat bit-identical.
Cases: both layouts, D = 64 and 128, ragged T (a partial last query block), with a sink per
head, a broadcast sink or none; inputs in range, guarded tails (q = k = sqrt(1000), the
reference's tail case), and single outliers placed so that each of the guard's three maxima
trips from one row owned by one workgroup (a large key at the last position, a large value at
the first, a NaN query in the middle). Workspaces start filled with NaN bytes, so no result
may depend on a zeroed workspace.
"""

import math

import numpy as np
import pytest

from helpers import attention_inputs

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

N_EXP, C = 16, 8.0


def _lib():
    from algebraic_amd import _lib
    return _lib


def _dirty_workspace(nbytes):
    return torch.full((nbytes,), 0xFF, dtype=torch.uint8, device="cuda")


def _clamp(T, n=N_EXP):
    t = 1e37 / (T + 1.0)
    for _ in range(int(math.log2(n))):
        t = math.sqrt(t)
    return 0.5 * (t - 1.0 / t)


def _two_calls(q, k, v, sink, nsink, layout, B, H, T, D, dt):
    L = _lib()
    lib = L.load()
    st = L.stream_of(q)
    ws_bytes = lib.alg_attn_workspace_size(dt, B, H, T, D)
    ws = _dirty_workspace(ws_bytes)
    q_s = torch.empty_like(q)
    sink_s = torch.full((H,), float("nan"), dtype=torch.float32, device="cuda")
    flag = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    L.check(lib.alg_attn_prepare(st, dt, B, H, T, D, L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(sink), nsink, C, N_EXP, 1,
                                 L.ptr(q_s), L.ptr(sink_s), L.ptr(flag), L.ptr(ws), ws_bytes), "prepare")
    o = torch.empty_like(q)
    stat = torch.empty((B, H, T), dtype=torch.float32, device="cuda")
    sink_arg = L.ptr(sink_s) if nsink else None  # sink/c exists only with a sink
    L.check(lib.alg_attn_fwd(st, dt, layout, B, H, T, D, L.ptr(q_s), L.ptr(k), L.ptr(v), sink_arg, N_EXP,
                             L.ATTN_GUARDED, L.ptr(flag), _clamp(T), 1, 1, L.ptr(o), None, L.ptr(stat)), "forward")
    torch.cuda.synchronize()
    return dict(q_s=q_s, sink_s=sink_s, flag=flag, o=o, stat=stat)


def _one_call(q, k, v, sink, nsink, layout, B, H, T, D, dt):
    L = _lib()
    lib = L.load()
    st = L.stream_of(q)
    ws_bytes = lib.alg_attn_workspace_size(dt, B, H, T, D)
    ws = _dirty_workspace(ws_bytes)
    q_s = torch.empty_like(q)
    sink_s = torch.full((H,), float("nan"), dtype=torch.float32, device="cuda")
    flag = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    o = torch.empty_like(q)
    stat = torch.empty((B, H, T), dtype=torch.float32, device="cuda")
    L.check(lib.alg_attn_fwd_guarded(st, dt, layout, B, H, T, D, L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(sink), nsink,
                                     C, N_EXP, L.ptr(q_s), L.ptr(sink_s), L.ptr(flag), L.ptr(o), None,
                                     L.ptr(stat), L.ptr(ws), ws_bytes), "alg_attn_fwd_guarded")
    torch.cuda.synchronize()
    return dict(q_s=q_s, sink_s=sink_s, flag=flag, o=o, stat=stat)


def _inputs(B, H, T, D, case, sink_kind, dtype, seed):
    q, k, v, _, s = attention_inputs(B, H, T, D, seed=seed, sink=sink_kind != "none")
    if case == "tail":  # test_flash_kernel_tpu.py:238-255: q = k = sqrt(1000)
        q = np.full_like(q, math.sqrt(1000.0))
        k = np.full_like(k, math.sqrt(1000.0))
    elif case == "big_key_last":
        k[-1, -1, T - 1, :] *= 1000.0
    elif case == "big_value_first":
        v[0, 0, 0, 0] = 1e30
    elif case == "nan_query_mid":
        q[B // 2, H // 2, T // 2, D // 3] = np.nan
    if sink_kind == "per_head":
        sink, nsink = s.reshape(-1), H
    elif sink_kind == "broadcast":
        sink, nsink = s.reshape(-1)[:1], 1
    else:
        sink, nsink = None, 0
    return q, k, v, sink, nsink


def _to_dev(a, layout, dtype):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if layout == 1:
        t = t.transpose(1, 2).contiguous()
    return t.to(device="cuda", dtype=dtype).contiguous()


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("case,sink_kind,shape", [
    ("in_range", "per_head", (2, 3, 200)),
    ("in_range", "broadcast", (1, 2, 640)),
    ("in_range", "none", (1, 2, 128)),
    ("tail", "per_head", (1, 2, 512)),
    ("tail", "none", (1, 1, 200)),
    ("big_key_last", "per_head", (2, 2, 200)),
    ("big_value_first", "none", (2, 2, 320)),
    ("nan_query_mid", "per_head", (2, 2, 256)),
])
def test_one_call_matches_prepare_then_forward(dtype, layout, D, case, sink_kind, shape):
    """f32 at D = 64 takes the same one-launch form (the f32 split forward forms q_s and the
    guard maxima); f32 at D = 128 is prepare + forward inside the call."""
    B, H, T = shape
    L = _lib()
    tdt, dt, bits = ((torch.bfloat16, L.DTYPE_BF16, torch.int16) if dtype == "bf16"
                     else (torch.float32, L.DTYPE_F32, torch.int32))
    q, k, v, sink, nsink = _inputs(B, H, T, D, case, sink_kind, tdt, seed=11 + T)
    qd, kd, vd = (_to_dev(a, layout, tdt) for a in (q, k, v))
    sd = None if sink is None else torch.from_numpy(np.ascontiguousarray(sink)).float().cuda()
    print(f"alg_attn_fwd_guarded {dtype} case={case} sink={sink_kind} B,H,T,D={B},{H},{T},{D} layout={layout}",
          flush=True)
    ref = _two_calls(qd, kd, vd, sd, nsink, layout, B, H, T, D, dt)
    got = _one_call(qd, kd, vd, sd, nsink, layout, B, H, T, D, dt)
    expect_flag = 1 if case == "in_range" else 0
    assert int(ref["flag"].item()) == expect_flag
    assert int(got["flag"].item()) == expect_flag
    assert torch.equal(got["q_s"].view(bits), ref["q_s"].view(bits))
    if nsink:
        assert torch.equal(got["sink_s"], ref["sink_s"])
    # Bit-identical outputs; NaN rows (the NaN-query case) compare as equal bit patterns.
    assert torch.equal(got["o"].view(bits), ref["o"].view(bits))
    assert torch.equal(got["stat"].view(torch.int32), ref["stat"].view(torch.int32))
    if case in ("in_range", "tail", "big_key_last"):
        assert torch.isfinite(got["o"].float()).all()


@pytest.mark.parametrize("case,sink_kind", [("in_range", "per_head"), ("tail", "none"), ("big_key_last", "per_head"),
                                            ("nan_query_mid", "broadcast")])
@pytest.mark.parametrize("T", [200, 256])
def test_one_call_f32_two_query_groups(case, sink_kind, T):
    """f32 at D = 64 with B H ceil(T/64) >= 512 takes the split forward's 64-query form (two
    query groups per workgroup, two-way key split, guard partials per 64-query block): its
    flag, q_s, o and stat are checked bit for bit against prepare + forward, and the flag
    against the expected branch, so a guard maximum it missed or misplaced fails here."""
    B, H, D, layout = 8, 16, 64, 0
    assert B * H * math.ceil(T / 64) >= 512
    L = _lib()
    q, k, v, sink, nsink = _inputs(B, H, T, D, case, sink_kind, torch.float32, seed=5 + T)
    qd, kd, vd = (_to_dev(a, layout, torch.float32) for a in (q, k, v))
    sd = None if sink is None else torch.from_numpy(np.ascontiguousarray(sink)).float().cuda()
    print(f"alg_attn_fwd_guarded f32 two query groups case={case} sink={sink_kind} T={T}", flush=True)
    ref = _two_calls(qd, kd, vd, sd, nsink, layout, B, H, T, D, L.DTYPE_F32)
    got = _one_call(qd, kd, vd, sd, nsink, layout, B, H, T, D, L.DTYPE_F32)
    expect_flag = 1 if case == "in_range" else 0
    assert int(ref["flag"].item()) == expect_flag
    assert int(got["flag"].item()) == expect_flag
    assert torch.equal(got["q_s"].view(torch.int32), ref["q_s"].view(torch.int32))
    if nsink:
        assert torch.equal(got["sink_s"], ref["sink_s"])
    assert torch.equal(got["o"].view(torch.int32), ref["o"].view(torch.int32))
    assert torch.equal(got["stat"].view(torch.int32), ref["stat"].view(torch.int32))
