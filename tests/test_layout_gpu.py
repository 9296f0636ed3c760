"""GPU parity of the projection-layout boundary: q, k, v, o, dO and the gradients stored
(B, T, H, D) (model.py:167-169, 182) give the same results as the reference's (B, H, T, D).

Only addressing differs between the two layouts (the same tiles, in the same order, feed the
same arithmetic), so bf16 results are compared bit for bit; the f32 path adds dq over key
blocks with atomics, whose order varies run to run, so its dq is compared at 1e-6.
The (B, H, T, D) results themselves are pinned to the oracle by test_attention_gpu.py,
test_prologue_gpu.py and test_full_size_gpu.py.
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
