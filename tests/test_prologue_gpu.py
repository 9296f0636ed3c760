"""GPU parity of the fused attention prologue (QK RMS norm + gain, Cayley rotation, q*alpha,
guard) and its VJP, through the host mirror and directly through the C ABI.

References: model.py:170-174 (composition), algebraic.py:76-83 (rms_norm), 124-179 (Cayley
tables, apply_rotary), flash.py:823-849 (prologue, guard). Oracle: oracle/prologue.py (pinned
by tests/test_prologue_oracle.py) chained with oracle/attention.py.
Bars (relative L2): bf16 1e-2 against the cast-faithful oracle chain and 2e-2 against torch
float64 autograd of the closed-form chain; f32 1e-5 (1e-4 for the gain gradients, sums over
every row); the two input layouts give bit-identical results.
"""

import math

import numpy as np
import pytest

from helpers import rel_l2
from oracle import attention as OA
from oracle import prologue as OP
from oracle.numerics import round_bf16

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

N_ATTN, C_ATTN = 16, 8.0


def _fn():
    from algebraic_amd.kernels.prologue import qk_norm_rotary_flash_attention
    return qk_norm_rotary_flash_attention


def _inputs(B, H, T, D, seed, dtype, gain=True, rotate=True, sink=True):
    rng = np.random.default_rng(seed)
    q, k, v, do = (rng.standard_normal((B, H, T, D)).astype(np.float32) for _ in range(4))
    q, k = q * 3.0, k * 0.6
    if dtype == "bf16":
        q, k, v, do = (round_bf16(a) for a in (q, k, v, do))
    gq = (1 + 0.2 * rng.standard_normal(D)).astype(np.float32) if gain else None
    gk = (1 + 0.2 * rng.standard_normal(D)).astype(np.float32) if gain else None
    cos, sin = OP.cayley_table_geometric(D, T) if rotate else (None, None)
    s = (rng.standard_normal((1, H, 1, 1)) * 0.1).astype(np.float32) if sink else None
    return q, k, v, do, s, gq, gk, cos, sin


def _oracle(q, k, v, do, sink, gq, gk, cos, sin, dtype):
    _, k_r, q_r, tau_q, tau_k = OP.prologue_forward(q, k, gq, gk, cos, sin, c=C_ATTN, dtype=dtype)
    res = OA.flash_attention_oracle(q_r, k_r, v, sink, do, n=N_ATTN, c=C_ATTN, dtype=dtype)
    assert res["in_range"]
    dq, dk, dgq, dgk = OP.prologue_backward(q, k, gq, gk, cos, sin, tau_q, tau_k, res["dq"], res["dk"], dtype=dtype)
    out = dict(o=res["o"], dq=dq, dk=dk, dv=res["dv"])
    if gq is not None:
        out.update(dq_gain=dgq, dk_gain=dgk)
    if sink is not None:
        out["dsink"] = res["dsink"]
    return out


def _run_hip(q, k, v, do, sink, gq, gk, cos, sin, dtype):
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    dev = lambda a: torch.tensor(a, device="cuda").to(tdt).requires_grad_(True)
    tq, tk, tv = dev(q), dev(k), dev(v)
    f32 = lambda a: None if a is None else torch.tensor(a, device="cuda", requires_grad=True)
    ts, tgq, tgk = f32(sink), f32(gq), f32(gk)
    tc = None if cos is None else torch.tensor(cos, device="cuda")
    tsn = None if sin is None else torch.tensor(sin, device="cuda")
    o = _fn()(tq, tk, tv, ts, tgq, tgk, tc, tsn, kind="asinh", n=N_ATTN, c=C_ATTN, range_guard=True,
              block=q.shape[2])
    o.backward(torch.tensor(do, device="cuda").to(tdt))
    torch.cuda.synchronize()
    g = lambda t: t.detach().float().cpu().numpy()
    out = dict(o=g(o), dq=g(tq.grad), dk=g(tk.grad), dv=g(tv.grad))
    if tgq is not None:
        out.update(dq_gain=g(tgq.grad), dk_gain=g(tgk.grad))
    if ts is not None:
        out["dsink"] = g(ts.grad)
    return out


def _compare(got, ref, tol, gain_tol=None, what=""):
    errs = {n: rel_l2(np.reshape(got[n], -1), np.reshape(ref[n], -1)) for n in ref}
    bad = {n: e for n, e in errs.items() if not e < (gain_tol if gain_tol and "gain" in n else tol)}
    assert not bad, f"{what}: {bad} (all {errs})"
    return errs


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("gain,rotate,sink", [(True, True, True), (False, True, False), (True, False, True)])
@pytest.mark.parametrize("shape", [(1, 2, 64, 64), (2, 2, 100, 128)])
def test_fused_prologue_attention_matches_oracle(shape, dtype, gain, rotate, sink):
    args = _inputs(*shape, seed=21, dtype=dtype, gain=gain, rotate=rotate, sink=sink)
    print(f"[prologue] {shape} {dtype} gain={gain} rotate={rotate} sink={sink}", flush=True)
    got = _run_hip(*args, dtype=dtype)
    ref = _oracle(*args, dtype=dtype)
    if dtype == "bf16":
        _compare(got, ref, 1e-2, what="HIP vs cast-faithful oracle")
    else:
        _compare(got, ref, 1e-5, gain_tol=1e-4, what="HIP vs f32 oracle")


def test_fused_prologue_attention_matches_torch_float64_chain():
    """bf16 HIP chain against torch float64 autograd of the closed forms."""
    from test_prologue_oracle import _torch_chain
    q, k, v, do, sink, gq, gk, cos, sin = _inputs(1, 2, 96, 64, seed=23, dtype="bf16")
    got = _run_hip(q, k, v, do, sink, gq, gk, cos, sin, "bf16")
    o, dq, dk, dv, dgq, dgk, ds = _torch_chain(q, k, v, do, sink, gq, gk, cos, sin)
    ref = dict(o=o, dq=dq, dk=dk, dv=dv, dq_gain=dgq, dk_gain=dgk, dsink=ds)
    _compare(got, ref, 2e-2, what="HIP bf16 vs float64 autograd")


# ---------------------------------------------------------------------------
# Direct C-ABI calls: layouts, tables, full size
# ---------------------------------------------------------------------------

def _lib():
    from algebraic_amd import _lib as L
    return L, L.load()


def _prologue_abi(q, k, v, gq, gk, cs, sn, layout, B, H, T, D, sink=None):
    """Forward prologue through the C ABI on device tensors stored in `layout` (q_s and k_r
    come back in it too)."""
    L, lib = _lib()
    dt = L.DTYPE_BF16 if q.dtype == torch.bfloat16 else L.DTYPE_F32
    q_s = torch.empty_like(q)
    k_r = torch.empty_like(q_s)
    tau_q = torch.empty((B, H, T), dtype=torch.float32, device="cuda")
    tau_k = torch.empty_like(tau_q)
    flag = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    sink_out = torch.empty(H, dtype=torch.float32, device="cuda") if sink is not None else None
    nbytes = lib.alg_attn_prologue_workspace_size(B, H, T, D)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    st = L.stream_of(q)
    L.check(lib.alg_attn_qk_prologue(st, dt, layout, B, H, T, D, L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(gq), L.ptr(gk),
                                      L.ptr(cs), L.ptr(sn), 1e-5, L.ptr(sink), 0 if sink is None else sink.numel(),
                                      C_ATTN, N_ATTN, 1, L.ptr(q_s), L.ptr(k_r), L.ptr(tau_q), L.ptr(tau_k),
                                      L.ptr(sink_out), L.ptr(flag), L.ptr(ws), nbytes), "prologue")
    torch.cuda.synchronize()
    return q_s, k_r, tau_q, tau_k, flag


def _prologue_bwd_abi(q, k, gq, gk, cs, sn, tau_q, tau_k, dq_r, dk_r, layout, B, H, T, D):
    L, lib = _lib()
    dt = L.DTYPE_BF16 if q.dtype == torch.bfloat16 else L.DTYPE_F32
    dq, dk = torch.empty_like(q), torch.empty_like(k)
    dgq = torch.empty(D, dtype=torch.float32, device="cuda") if gq is not None else None
    dgk = torch.empty(D, dtype=torch.float32, device="cuda") if gk is not None else None
    nbytes = lib.alg_attn_prologue_workspace_size(B, H, T, D)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    L.check(lib.alg_attn_qk_prologue_bwd(L.stream_of(q), dt, layout, B, H, T, D, L.ptr(q), L.ptr(k), L.ptr(gq),
                                          L.ptr(gk), L.ptr(cs), L.ptr(sn), L.ptr(tau_q), L.ptr(tau_k), L.ptr(dq_r),
                                          L.ptr(dk_r), L.ptr(dq), L.ptr(dk), L.ptr(dgq), L.ptr(dgk), L.ptr(ws),
                                          nbytes), "prologue bwd")
    torch.cuda.synchronize()
    return dq, dk, dgq, dgk


def _bthd(x):
    return x.permute(0, 2, 1, 3).contiguous()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_prologue_layouts_agree_bitwise(dtype):
    """(B,T,H,D) storage of the raw projections gives bit-identical outputs and gradients."""
    L, _ = _lib()
    B, H, T, D = 2, 3, 80, 128
    g = torch.Generator(device="cuda")
    g.manual_seed(3)
    rn = lambda *s: torch.randn(*s, device="cuda", generator=g)
    q, k, v = (rn(B, H, T, D).to(dtype) for _ in range(3))
    gq, gk = 1 + 0.2 * rn(D), 1 + 0.2 * rn(D)
    w = torch.tensor(OP.geometric_frequencies(D), device="cuda")
    from algebraic_amd.kernels.prologue import cayley_powers
    cs, sn = cayley_powers(w, T)
    a = _prologue_abi(q, k, v, gq, gk, cs, sn, L.LAYOUT_BHTD, B, H, T, D)
    b = _prologue_abi(_bthd(q), _bthd(k), _bthd(v), gq, gk, cs, sn, L.LAYOUT_BTHD, B, H, T, D)
    assert torch.equal(_bthd(a[0]), b[0]) and torch.equal(_bthd(a[1]), b[1])  # q_s, k_r in the layout
    for x, y in zip(a[2:], b[2:]):  # 1/rms rows (B, H, T) and the guard flag
        assert torch.equal(x, y)
    dq_r, dk_r = rn(B, H, T, D).to(dtype), rn(B, H, T, D).to(dtype)
    da = _prologue_bwd_abi(q, k, gq, gk, cs, sn, a[2], a[3], dq_r, dk_r, L.LAYOUT_BHTD, B, H, T, D)
    db = _prologue_bwd_abi(_bthd(q), _bthd(k), gq, gk, cs, sn, b[2], b[3], _bthd(dq_r), _bthd(dk_r),
                           L.LAYOUT_BTHD, B, H, T, D)
    assert torch.equal(_bthd(da[0]), db[0]) and torch.equal(_bthd(da[1]), db[1])
    assert torch.equal(da[2], db[2]) and torch.equal(da[3], db[3])


@pytest.mark.parametrize("head_dim,T", [(64, 300), (128, 2048)])
def test_cayley_tables_are_exact_rotations(head_dim, T):
    """Device tables against cos/sin(m 2 atan w) with the reference's bound
    (tests/test_components.py:59-68: 2e-5 at T = 300; the oracle's pin allows 2e-4 at
    T = 2048, where one-ulp differences in the binary powers grow with m), unit norm, and the
    NumPy restatement within the same bound."""
    from algebraic_amd.kernels.prologue import cayley_table_geometric
    c, s = (t.cpu().numpy() for t in cayley_table_geometric(head_dim, T))
    half = head_dim // 2
    angles = 2 * np.arctan(0.5 * 1e4 ** (-np.arange(half) / half))
    m = np.arange(T)[:, None]
    tol = 2e-5 if T <= 300 else 2e-4
    np.testing.assert_allclose(c, np.cos(m * angles), atol=tol)
    np.testing.assert_allclose(s, np.sin(m * angles), atol=tol)
    np.testing.assert_allclose(c * c + s * s, 1.0, atol=1e-6)
    c_ref, s_ref = OP.cayley_table_geometric(head_dim, T)
    print(f"  max |device - oracle|: cos {np.max(np.abs(c - c_ref)):.2e} sin {np.max(np.abs(s - s_ref)):.2e}")
    np.testing.assert_allclose(c, c_ref, atol=tol)
    np.testing.assert_allclose(s, s_ref, atol=tol)


def test_prologue_full_size_c4a():
    """C4a shape (B8 H16 T2048 D128, bf16, projection layout (B,T,H,D)): forward outputs and
    the VJP (random cotangents) of every row against the oracle."""
    L, _ = _lib()
    B, H, T, D = 8, 16, 2048, 128
    rng = np.random.default_rng(31)
    q, k, v, dq_r, dk_r = (round_bf16(rng.standard_normal((B, H, T, D)).astype(np.float32)) for _ in range(5))
    q, k = round_bf16(q * 3.0), round_bf16(k * 0.6)
    gq = (1 + 0.2 * rng.standard_normal(D)).astype(np.float32)
    gk = (1 + 0.2 * rng.standard_normal(D)).astype(np.float32)
    cos, sin = OP.cayley_table_geometric(D, T)
    print("[prologue] full size C4a", flush=True)
    dev = lambda a: torch.tensor(a, device="cuda").to(torch.bfloat16)
    tq, tk, tv = dev(q), dev(k), dev(v)
    f = lambda a: torch.tensor(a, device="cuda")
    q_s, k_r, tau_q, tau_k, flag = _prologue_abi(_bthd(tq), _bthd(tk), _bthd(tv), f(gq), f(gk), f(cos), f(sin),
                                                 L.LAYOUT_BTHD, B, H, T, D)
    r_qs, r_kr, _, r_tq, r_tk = OP.prologue_forward(q, k, gq, gk, cos, sin, c=C_ATTN, dtype="bf16")
    np_ = lambda t: t.float().cpu().numpy()
    q_s, k_r = q_s.permute(0, 2, 1, 3), k_r.permute(0, 2, 1, 3)  # (B, T, H, D) -> (B, H, T, D)
    errs = {"q_s": rel_l2(np_(q_s), r_qs), "k_r": rel_l2(np_(k_r), r_kr),
            "tau_q": rel_l2(np_(tau_q), r_tq), "tau_k": rel_l2(np_(tau_k), r_tk)}
    print(f"  forward: {errs}", flush=True)
    assert max(errs.values()) < 1e-3, errs
    assert int(flag.item()) == int(OA.guard_in_range(r_qs, r_kr, v, np.zeros(1, np.float32), has_sink=False))
    dq, dk, dgq, dgk = _prologue_bwd_abi(_bthd(tq), _bthd(tk), f(gq), f(gk), f(cos), f(sin), tau_q, tau_k,
                                         _bthd(dev(dq_r)), _bthd(dev(dk_r)), L.LAYOUT_BTHD, B, H, T, D)
    r_dq, r_dk, r_dgq, r_dgk = OP.prologue_backward(q, k, gq, gk, cos, sin, r_tq, r_tk, dq_r, dk_r, dtype="bf16")
    errs = {"dq": rel_l2(np_(dq).transpose(0, 2, 1, 3), r_dq), "dk": rel_l2(np_(dk).transpose(0, 2, 1, 3), r_dk),
            "dq_gain": rel_l2(np_(dgq), r_dgq), "dk_gain": rel_l2(np_(dgk), r_dgk)}
    print(f"  backward: {errs}", flush=True)
    assert max(errs.values()) < 1e-3, errs
