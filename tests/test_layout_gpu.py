"""GPU parity of the projection-layout boundary: q, k, v, o, dO and the gradients stored
(B, T, H, D) (model.py:167-169, 182) give the same results as the reference's (B, H, T, D).

Only addressing differs between the two layouts (the same tiles, in the same order, feed the
same arithmetic), so bf16 results are compared bit for bit; the f32 path adds dq over key
blocks with atomics, whose order varies run to run, so its dq is compared at 1e-6.
The (B, T, H, D) results are also compared with the oracle directly (dense float64 and the
cast-faithful kernel restatement) for the guarded, shifted-fallback, clipped and explicitly
shifted variants, ragged T included.
"""

import math

import numpy as np
import pytest

from helpers import attention_inputs

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _bthd(x):
    return x.permute(0, 2, 1, 3).contiguous()


def _run(fn, q, k, v, sink, do, **kw):
    tq, tk, tv = (a.clone().requires_grad_(True) for a in (q, k, v))
    ts = None if sink is None else sink.clone().requires_grad_(True)
    o = fn(tq, tk, tv, ts, **kw)
    o.backward(do)
    torch.cuda.synchronize()
    out = [o.detach(), tq.grad, tk.grad, tv.grad]
    if ts is not None:
        out.append(ts.grad)
    return out


def _check_layouts(fn, q, k, v, sink, do, exact=True, **kw):
    a = _run(fn, q, k, v, sink, do, layout="bhtd", **kw)
    b = _run(fn, _bthd(q), _bthd(k), _bthd(v), sink, _bthd(do), layout="bthd", **kw)
    names = ["o", "dq", "dk", "dv", "dsink"]
    for name, x, y in zip(names, a, b):
        y = y if name == "dsink" else _bthd(y)  # (B, T, H, D) -> (B, H, T, D)
        if exact or name not in ("dq", "dsink"):
            assert torch.equal(x, y), f"{name} differs between layouts"
        else:
            err = float((x.float() - y.float()).norm() / x.float().norm().clamp_min(1e-30))
            assert err < 1e-6, f"{name}: {err}"


def _dev(a, dtype):
    return torch.tensor(a, device="cuda").to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(2, 3, 100, 64), (1, 2, 160, 128)])
def test_flash_layouts_agree(shape, dtype):
    from algebraic_amd.kernels.flash import flash_attention
    q, k, v, do, sink = attention_inputs(*shape, seed=41, dtype="bf16" if dtype == torch.bfloat16 else "f32")
    print(f"[layout] flash {shape} {dtype}", flush=True)
    _check_layouts(flash_attention, _dev(q, dtype), _dev(k, dtype), _dev(v, dtype),
                   torch.tensor(sink, device="cuda"), _dev(do, dtype), exact=dtype == torch.bfloat16,
                   kind="asinh", n=16, c=8.0, block=shape[2], range_guard=True)


@pytest.mark.parametrize("variant", ["shifted_fallback", "explicit_shift", "clipped"])
def test_flash_layouts_agree_other_variants(variant):
    """The guard's shifted fallback (forced by large scores), explicit shift=True and the
    clipped unguarded default, bf16."""
    from algebraic_amd.kernels.flash import flash_attention
    shape = (1, 2, 96, 64)
    scale = 12.0 if variant == "shifted_fallback" else 1.0
    q, k, v, do, sink = attention_inputs(*shape, seed=43, dtype="bf16", scale=scale)
    kw = dict(kind="asinh", n=16, c=8.0, block=96)
    if variant == "shifted_fallback":
        kw["range_guard"] = True
    elif variant == "explicit_shift":
        kw["shift"] = True
    print(f"[layout] {variant}", flush=True)
    t = lambda a: _dev(a, torch.bfloat16)
    _check_layouts(flash_attention, t(q), t(k), t(v), torch.tensor(sink, device="cuda"), t(do), **kw)


def test_prologue_flash_layouts_agree():
    from algebraic_amd.kernels.prologue import qk_norm_rotary_flash_attention, cayley_table_geometric
    B, H, T, D = 2, 2, 128, 128
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    rn = lambda *s: torch.randn(*s, device="cuda", generator=g)
    q, k, v, do = (rn(B, H, T, D).to(torch.bfloat16) for _ in range(4))
    gq, gk = (1 + 0.2 * rn(D)).requires_grad_(True), (1 + 0.2 * rn(D)).requires_grad_(True)
    cs, sn = cayley_table_geometric(D, T)
    sink = 0.1 * rn(1, H, 1, 1)
    print("[layout] fused prologue", flush=True)

    def fn(tq, tk, tv, ts, layout):
        return qk_norm_rotary_flash_attention(tq, tk, tv, ts, gq, gk, cs, sn, kind="asinh", n=16, c=8.0, block=T,
                                              range_guard=True, layout=layout)
    a = _run(fn, q, k, v, sink, do, layout="bhtd")
    ga = (gq.grad.clone(), gk.grad.clone())
    gq.grad = gk.grad = None
    b = _run(fn, _bthd(q), _bthd(k), _bthd(v), sink, _bthd(do), layout="bthd")
    for name, x, y in zip(["o", "dq", "dk", "dv"], a, b):
        assert torch.equal(x, _bthd(y)), f"{name} differs between layouts"
    assert torch.equal(a[4], b[4])
    assert torch.equal(ga[0], gq.grad) and torch.equal(ga[1], gk.grad)


def test_flash_layouts_agree_full_size_c4a():
    """C4a (B8 H16 T2048 D128 bf16) in both layouts: bit-identical, and the (B, T, H, D)
    output is the (B, T, H*D) projection input as a view."""
    from algebraic_amd.kernels.flash import flash_attention
    B, H, T, D = 8, 16, 2048, 128
    g = torch.Generator(device="cuda")
    g.manual_seed(9)
    rn = lambda *s: torch.randn(*s, device="cuda", generator=g)
    norm = lambda x: x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-5)
    q, k = (norm(rn(B, H, T, D)).to(torch.bfloat16) for _ in range(2))
    v, do = (rn(B, H, T, D).to(torch.bfloat16) for _ in range(2))
    sink = 0.1 * rn(1, H, 1, 1)
    print("[layout] full size C4a", flush=True)
    kw = dict(kind="asinh", n=16, c=8.0, block=512, range_guard=True)
    _check_layouts(flash_attention, q, k, v, sink, do, **kw)
    o = flash_attention(_bthd(q), _bthd(k), _bthd(v), sink, layout="bthd", **kw)
    flat = o.reshape(B, T, H * D)
    assert flat.data_ptr() == o.data_ptr() and flat.is_contiguous()


# ---------------------------------------------------------------------------
# (B, T, H, D) storage against the oracle itself (model.py:167-169, 182 feed attention the
# projection layout): the inputs are drawn (B, H, T, D), stored (B, T, H, D) on the device,
# and every output and gradient, read back into (B, H, T, D), is compared with the float64
# dense oracle (algebraic.py:186-216) and, for the guarded path, with the cast-faithful
# restatement of the kernels (flash.py:763-857).
# ---------------------------------------------------------------------------
BF16_DENSE, BF16_KERNEL, F32_DENSE = 2e-2, 1e-2, 1e-5


def _np_bthd(a):
    return np.ascontiguousarray(np.transpose(a, (0, 2, 1, 3)))


def _run_bthd(q, k, v, do, sink, dtype, **kw):
    from algebraic_amd.kernels.flash import flash_attention
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    dev = lambda a: torch.tensor(_np_bthd(a), device="cuda").to(tdt)
    tq, tk, tv = (dev(a).requires_grad_(True) for a in (q, k, v))
    ts = None if sink is None else torch.tensor(sink, device="cuda", requires_grad=True)
    o = flash_attention(tq, tk, tv, ts, kind="asinh", n=16, c=8.0, layout="bthd", **kw)
    assert o.shape == tq.shape  # (B, T, H, D)
    o.backward(dev(do))
    torch.cuda.synchronize()
    back = lambda t: np.transpose(t.detach().float().cpu().numpy().astype(np.float64), (0, 2, 1, 3))
    out = [back(o), back(tq.grad), back(tk.grad), back(tv.grad)]
    out.append(None if ts is None else ts.grad.detach().cpu().numpy().astype(np.float64))
    return out


def _check_dense(res, q, k, v, do, sink, tol):
    from helpers import rel_l2
    from oracle import attention as OA
    want = [OA.dense_forward(q, k, v, sink, n=16, c=8.0), *OA.dense_backward(q, k, v, sink, do, n=16, c=8.0)]
    names = ["o", "dq", "dk", "dv", "dsink"]
    errs = {nm: rel_l2(a, b) for nm, a, b in zip(names, res, want) if b is not None and a is not None}
    bad = {nm: e for nm, e in errs.items() if not e < tol}
    assert not bad, f"(B, T, H, D) vs dense oracle: {bad} (all {errs})"


def _check_kernel(res, q, k, v, do, sink, dtype, tol, in_range):
    from helpers import rel_l2
    from oracle import attention as OA
    ref = OA.flash_attention_oracle(q, k, v, sink, do, n=16, c=8.0, dtype=dtype)
    assert ref["in_range"] == in_range
    names = ["o", "dq", "dk", "dv", "dsink"]
    errs = {nm: rel_l2(a, ref[nm]) for nm, a in zip(names, res) if a is not None and nm in ref}
    bad = {nm: e for nm, e in errs.items() if not e < tol}
    assert not bad, f"(B, T, H, D) vs kernel restatement: {bad} (all {errs})"


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("shape", [(2, 3, 100, 64), (1, 2, 160, 128), (2, 2, 33, 128)])
@pytest.mark.parametrize("with_sink", [True, False])
def test_bthd_guarded_matches_oracle(shape, dtype, with_sink):
    """Guarded path in range (the model's call), ragged T included."""
    from helpers import attention_inputs
    q, k, v, do, sink = attention_inputs(*shape, seed=47, dtype=dtype, sink=with_sink)
    print(f"[layout-oracle] guarded {shape} {dtype} sink={with_sink}", flush=True)
    res = _run_bthd(q, k, v, do, sink, dtype, range_guard=True, block=shape[2])
    _check_dense(res, q, k, v, do, sink, BF16_DENSE if dtype == "bf16" else F32_DENSE)
    if dtype == "bf16":
        _check_kernel(res, q, k, v, do, sink, dtype, BF16_KERNEL, in_range=True)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_bthd_shifted_fallback_matches_oracle(dtype):
    """Scores past the guard's bound (q, k x 5: ||q_s||^2 ||k||^2 = 5^4 D / 64 > (16/1.01)^2)
    take the shifted fallback chosen on the device."""
    from helpers import attention_inputs
    shape = (2, 3, 100, 64)
    q, k, v, do, sink = attention_inputs(*shape, seed=53, dtype=dtype, scale=5.0)
    print(f"[layout-oracle] shifted fallback {shape} {dtype}", flush=True)
    res = _run_bthd(q, k, v, do, sink, dtype, range_guard=True, block=shape[2])
    _check_dense(res, q, k, v, do, sink, BF16_DENSE if dtype == "bf16" else 1e-4)
    _check_kernel(res, q, k, v, do, sink, dtype, BF16_KERNEL if dtype == "bf16" else 1e-4, in_range=False)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("variant", ["clipped", "explicit_shift"])
def test_bthd_unguarded_variants_match_dense(variant, dtype):
    """range_guard=False (the clipped unshifted default, flash.py:749-754) and shift=True."""
    from helpers import attention_inputs
    shape = (1, 2, 160, 128) if variant == "clipped" else (2, 3, 100, 64)
    q, k, v, do, sink = attention_inputs(*shape, seed=59, dtype=dtype)
    kw = dict(range_guard=False, block=32) if variant == "clipped" else dict(shift=True, block=shape[2])
    print(f"[layout-oracle] {variant} {shape} {dtype}", flush=True)
    res = _run_bthd(q, k, v, do, sink, dtype, **kw)
    _check_dense(res, q, k, v, do, sink, BF16_DENSE if dtype == "bf16" else F32_DENSE)
