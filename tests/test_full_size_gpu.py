"""GPU parity at the BASELINE.json full sizes (C1 is covered in test_attention_gpu.py).

* C3  attention fwd+bwd bf16 B8 H16 T2048 D64
* C4a attention fwd+bwd bf16 B8 H16 T2048 D128
* C5  attention (long context) bf16 B1 H16 T16384 D128
* C2  head fwd+bwd N8192 d768 V50257
* C4b head fwd+bwd N16384 d2048 V32000

At these sizes every output and gradient of the HIP path is compared element by element with
the float32 torch restatement of the same cast-faithful maths (tests/torch_ref.py, pinned to
the NumPy oracle on the CPU by tests/test_torch_ref.py and here on sampled heads / tokens),
and sampled heads, rows and tokens are compared directly with the NumPy oracle (cast-faithful
kernel restatement, and the float64 dense oracle for one attention head). Size-independent
properties close the loop: causality (perturbing keys and values at positions >= p leaves the
output and dq of every row < p bit-identical) and row normalisation (v = 1, no sink: every
output is 1 up to the bf16 rounding of the weights and of the output).

Bars (relative L2 per tensor; per (b,h) head as well for attention): 1e-2 against the
cast-faithful restatements (torch and NumPy), 2e-2 against the float64 dense oracle (the
north-star bf16 bar), 2e-3 between the two restatements.
Inputs follow the distributions of the configs (Q/K/V/dO ~ N(0,1) with Q, K RMS-normalised,
sink ~ N(0, 0.1); h RMS-normalised N(0,1), E ~ N(0, 0.02), uniform targets), seeded NumPy.
"""

import numpy as np
import pytest

from helpers import attention_inputs, head_inputs, rel_l2
from oracle import attention as OA
from oracle import head as OH

torch = pytest.importorskip("torch")
import torch_ref  # noqa: E402

pytestmark = pytest.mark.gpu

KERNEL, DENSE, REFS = 1e-2, 2e-2, 2e-3
N_ATTN, C_ATTN, N_HEAD, C_HEAD = 16, 8.0, 8, 2.0
ATTN_CONFIGS = {"C3": (8, 16, 2048, 64), "C4a": (8, 16, 2048, 128)}
C5 = (1, 16, 16384, 128)
HEAD_CONFIGS = {"C2": (8192, 768, 50257), "C4b": (16384, 2048, 32000)}


@pytest.fixture(autouse=True)
def _fp32_products():
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    yield
    torch.backends.cuda.matmul.allow_tf32 = prev


def _flash():
    from algebraic_amd.kernels.flash import flash_attention
    return flash_attention


def _dev(a, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def _np(t):
    return t.detach().float().cpu().numpy()


def _run_attention(q, k, v, sink, do):
    """Guarded flash_attention forward (+ backward when ``do`` is given) on device tensors."""
    tq, tk, tv = (a.clone().requires_grad_(do is not None) for a in (q, k, v))
    ts = None if sink is None else sink.clone().requires_grad_(do is not None)
    o = _flash()(tq, tk, tv, ts, kind="asinh", n=N_ATTN, c=C_ATTN, block=512, range_guard=True)
    out = {"o": o.detach().float()}
    if do is not None:
        o.backward(do)
        out.update(dq=tq.grad.float(), dk=tk.grad.float(), dv=tv.grad.float())
        if ts is not None:
            out["dsink"] = ts.grad.reshape(-1).float()
    torch.cuda.synchronize()
    return out


def _per_head_rel_l2(a, b):
    """Largest relative L2 error over the (b,h) heads of two (B,H,T,D) device tensors."""
    num = (a - b).flatten(2).norm(dim=-1)
    den = b.flatten(2).norm(dim=-1).clamp_min(1e-30)
    return float((num / den).max())


def _assert_close(errs, bar, what):
    print(f"  {what}: " + ", ".join(f"{key}={val:.2e}" for key, val in errs.items()), flush=True)
    bad = {key: val for key, val in errs.items() if not val < bar}
    assert not bad, f"{what}: {bad} over the bar {bar} (all {errs})"


def _attention_case(shape, backward, seed=1):
    B, H, T, D = shape
    q, k, v, do, sink = attention_inputs(B, H, T, D, seed=seed, dtype="bf16")
    q_s, beta, alpha = OA.prologue(q, sink, c=C_ATTN, dtype="bf16")
    assert OA.guard_in_range(q_s, k, v, beta, n=N_ATTN), "config inputs must take the in-range branch"
    dev = dict(q=_dev(q), k=_dev(k), v=_dev(v), do=_dev(do) if backward else None,
               sink=torch.from_numpy(sink).to("cuda"))
    return (q, k, v, do, sink, q_s, beta, alpha), dev


@pytest.mark.parametrize("config", list(ATTN_CONFIGS))
def test_attention_full_size(config):
    B, H, T, D = shape = ATTN_CONFIGS[config]
    (q, k, v, do, sink, q_s, beta, alpha), dev = _attention_case(shape, backward=True)
    print(f"[full-size] attention {config} {shape}", flush=True)
    hip = _run_attention(dev["q"], dev["k"], dev["v"], dev["sink"], dev["do"])
    ref = torch_ref.attention(dev["q"], dev["k"], dev["v"], dev["sink"], dev["do"], n=N_ATTN, c=C_ATTN)

    # Every element at full size against the torch restatement.
    errs = {name: rel_l2(_np(hip[name]), _np(ref[name])) for name in ("o", "dq", "dk", "dv", "dsink")}
    errs.update({f"{name}/head": _per_head_rel_l2(hip[name], ref[name]) for name in ("o", "dq", "dk", "dv")})
    _assert_close(errs, KERNEL, f"{config}: HIP vs float32 restatement")

    # Sampled heads against the NumPy oracle (cast-faithful kernel restatement).
    heads = [(0, 0), (B - 1, H - 1), (B // 2, H // 3)]
    o_np, stat_np, _ = OA.kernel_forward(q_s, k, v, beta, n=N_ATTN, dtype="bf16", heads=heads)
    dq_s, dk_np, dv_np, _, _, dq_np = OA.kernel_backward(q_s, k, v, beta, o_np, stat_np, do, n=N_ATTN,
                                                          alpha=alpha, dtype="bf16", heads=heads)
    oracle = dict(o=o_np, dq=dq_np, dk=dk_np, dv=dv_np)
    for b, h in heads:
        e_hip = {n: rel_l2(_np(hip[n][b, h]), oracle[n][b, h]) for n in oracle}
        _assert_close(e_hip, KERNEL, f"{config}: HIP vs NumPy oracle at head ({b},{h})")
        e_ref = {n: rel_l2(_np(ref[n][b, h]), oracle[n][b, h]) for n in oracle}
        e_ref["stat"] = rel_l2(_np(ref["stat"][b, h]), stat_np[b, h])
        _assert_close(e_ref, REFS, f"{config}: float32 restatement vs NumPy oracle at head ({b},{h})")

    # One head against the float64 dense oracle (the reference's non-kernel path).
    b, h = heads[-1]
    sl = (slice(b, b + 1), slice(h, h + 1))
    s_h = sink[:, h:h + 1]
    o_d = OA.dense_forward(q[sl], k[sl], v[sl], s_h, n=N_ATTN, c=C_ATTN)
    dq_d, dk_d, dv_d, _ = OA.dense_backward(q[sl], k[sl], v[sl], s_h, do[sl], n=N_ATTN, c=C_ATTN)
    e_dense = {"o": rel_l2(_np(hip["o"][b, h]), o_d[0, 0]), "dq": rel_l2(_np(hip["dq"][b, h]), dq_d[0, 0]),
               "dk": rel_l2(_np(hip["dk"][b, h]), dk_d[0, 0]), "dv": rel_l2(_np(hip["dv"][b, h]), dv_d[0, 0])}
    _assert_close(e_dense, DENSE, f"{config}: HIP vs float64 dense oracle at head ({b},{h})")


def test_attention_long_context_c5():
    """C5: forward (the config's pass) and backward at T = 16384 against the torch
    restatement, and sampled rows of two heads against the NumPy oracle."""
    B, H, T, D = C5
    (q, k, v, do, sink, q_s, beta, alpha), dev = _attention_case(C5, backward=True, seed=4)
    print(f"[full-size] attention C5 {C5}", flush=True)
    hip = _run_attention(dev["q"], dev["k"], dev["v"], dev["sink"], dev["do"])
    ref = torch_ref.attention(dev["q"], dev["k"], dev["v"], dev["sink"], dev["do"], n=N_ATTN, c=C_ATTN,
                              heads_per_chunk=1)
    errs = {name: rel_l2(_np(hip[name]), _np(ref[name])) for name in ("o", "dq", "dk", "dv", "dsink")}
    errs.update({f"{name}/head": _per_head_rel_l2(hip[name], ref[name]) for name in ("o", "dq", "dk", "dv")})
    _assert_close(errs, KERNEL, "C5: HIP vs float32 restatement")

    rng = np.random.default_rng(11)
    rows = np.unique(np.concatenate([[0, 1, 31, 32, 63, 64, 127, 128, 4095, 8191, T - 2, T - 1],
                                     rng.integers(0, T, 20)]))
    heads = [(0, 0), (0, H - 1)]
    o_np, stat_np, _ = OA.kernel_forward(q_s, k, v, beta, n=N_ATTN, dtype="bf16", heads=heads, rows=rows)
    for b, h in heads:
        e = {"o": rel_l2(_np(hip["o"][b, h])[rows], o_np[b, h, rows]),
             "o/ref": rel_l2(_np(ref["o"][b, h])[rows], o_np[b, h, rows]),
             "stat/ref": rel_l2(_np(ref["stat"][b, h])[rows], stat_np[b, h, rows])}
        _assert_close(e, KERNEL, f"C5: sampled rows of head ({b},{h}) vs NumPy oracle")
        _assert_close({k: e[k] for k in ("o/ref", "stat/ref")}, REFS, "C5: float32 restatement vs NumPy oracle")


def test_attention_causality_full_size():
    """C4a shape: keys and values at positions >= p do not reach rows < p (forward output and
    dq are bit-identical), while later rows do change."""
    B, H, T, D = ATTN_CONFIGS["C4a"]
    (q, k, v, do, sink, *_), dev = _attention_case((B, H, T, D), backward=True, seed=6)
    print("[full-size] causality C4a", flush=True)
    first = _run_attention(dev["q"], dev["k"], dev["v"], dev["sink"], dev["do"])
    p = T // 2 + 37
    q2, k2, v2, *_ = attention_inputs(B, H, T, D, seed=7, dtype="bf16")
    k_new, v_new = dev["k"].clone(), dev["v"].clone()
    k_new[:, :, p:] = _dev(k2[:, :, p:])
    v_new[:, :, p:] = _dev(v2[:, :, p:])
    second = _run_attention(dev["q"], k_new, v_new, dev["sink"], dev["do"])
    for name in ("o", "dq"):
        assert torch.equal(first[name][:, :, :p], second[name][:, :, :p]), f"{name} rows < {p} changed"
        assert not torch.equal(first[name][:, :, p:], second[name][:, :, p:]), f"{name} rows >= {p} unchanged"


def test_attention_rows_normalised_long_context():
    """C5 shape, v = 1 and no sink: o_i = sum_j round(w_ij) / sum_j w_ij = 1 within the bf16
    rounding of the weights (2^-9 relative) and of the output (2^-8)."""
    B, H, T, D = C5
    q, k, _, _, _ = attention_inputs(B, H, T, D, seed=8, dtype="bf16", sink=False)
    print("[full-size] row normalisation C5", flush=True)
    ones = torch.ones((B, H, T, D), dtype=torch.bfloat16, device="cuda")
    out = _run_attention(_dev(q), _dev(k), ones, None, None)
    err = float((out["o"] - 1.0).abs().max())
    print(f"  C5 row normalisation: max |o - 1| = {err:.2e}", flush=True)
    assert err <= 2.0 ** -9 + 2.0 ** -8, f"max |o - 1| = {err}"


@pytest.mark.parametrize("schedule", ["residual", "streamed"])
@pytest.mark.parametrize("config", list(HEAD_CONFIGS))
def test_head_full_size(config, schedule, monkeypatch):
    """The default (residual) schedule and the streamed one at its default vocabulary chunk."""
    from algebraic_amd.kernels import fused_head as FH
    from algebraic_amd.kernels.fused_head import fused_head
    monkeypatch.setattr(FH, "SCHEDULE", schedule)
    monkeypatch.setattr(FH, "VOCAB_CHUNK", 0)
    N, d, V = shape = HEAD_CONFIGS[config]
    h, E, tg = head_inputs(N, d, V, seed=2)
    print(f"[full-size] head {config} {shape} {schedule}", flush=True)
    th = _dev(h).requires_grad_(True)
    tE = _dev(E).requires_grad_(True)
    tt = torch.from_numpy(tg).to("cuda")
    obj, tel = fused_head(th, tE, tt, kind="alg_ce", n=N_HEAD, c=C_HEAD)
    obj.backward()
    torch.cuda.synchronize()
    ref = torch_ref.head(th.detach(), tE.detach(), tt, 1.0, n=N_HEAD, c=C_HEAD)
    errs = {"obj": abs(float(obj.detach()) - float(ref["obj"])) / abs(float(ref["obj"])),
            "pt": rel_l2(_np(tel), _np(ref["pt"])),
            "dh": rel_l2(_np(th.grad), _np(ref["dh"])), "dE": rel_l2(_np(tE.grad), _np(ref["dE"]))}
    _assert_close(errs, KERNEL, f"{config}: HIP vs float32 restatement")

    rng = np.random.default_rng(12)
    toks = np.unique(np.concatenate([[0, 1, 255, 256, N - 1], rng.integers(0, N, 59)]))
    stat_np, _, pt_np, _ = OH.kernel_forward(h, E, tg, n=N_HEAD, c=C_HEAD, rows=toks)
    dh_np, _ = OH.kernel_backward(h, E, tg, stat_np, 1.0, n=N_HEAD, c=C_HEAD, rows=toks)
    e = {"pt": rel_l2(_np(tel)[toks], pt_np[toks]), "dh": rel_l2(_np(th.grad)[toks], dh_np[toks])}
    _assert_close(e, KERNEL, f"{config}: sampled tokens, HIP vs NumPy oracle")
    e_ref = {"stat": rel_l2(_np(ref["stat"])[toks], stat_np[toks]), "pt": rel_l2(_np(ref["pt"])[toks], pt_np[toks]),
             "dh": rel_l2(_np(ref["dh"])[toks], dh_np[toks])}
    _assert_close(e_ref, REFS, f"{config}: sampled tokens, float32 restatement vs NumPy oracle")
